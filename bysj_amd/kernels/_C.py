"""Native entry points of the operator slice over the libdpa4k C ABI.

This module takes the place of the reference's pybind module ``kernels._C``
(csrc/bindings.cpp:6-29): the same nine symbols with the same positional and
keyword arguments, returning the same tuples.  Each entry point re-checks its
tensors the way the reference's ``TORCH_CHECK`` host launchers do (raising
``RuntimeError``), allocates the outputs and any workspace with torch on the
tensors' device, and enqueues the HIP kernels on the current torch stream
through ctypes.  There is no CPU path: importing this module fails when
libdpa4k.so has not been built.

Extensions over the reference, all keyword-only or additional symbols:
``segment_sum_backward(..., want_edge_scale_grad=True)`` returns a third
tensor, the ``edge_scale`` gradient; ``force_assembly`` also takes float64
inputs; ``segment_offsets``, ``group_by_key``, ``gie_group`` and the
``*_csr`` GIE entry points expose the device-side CSR construction;
``segment_softmax_plan`` builds the degree plan that
``segment_softmax_forward/backward(..., plan=...)`` accept;
``gie_rmsnorm_forward_csr`` is the fused GIE -> RMSNorm forward;
``edge_stream_combine`` is the fused edge-stream elementwise chain.
"""
from __future__ import annotations

import ctypes
import weakref

import torch

from . import _lib

_LIB = _lib.load()


# ---------------------------------------------------------------------------
# checks (restating csrc/checks.h:6-20 and the per-op TORCH_CHECKs)
# ---------------------------------------------------------------------------

def _check(condition: bool, message: str) -> None:
    if not condition:
        raise RuntimeError(message)


def _f32(tensor, what: str) -> None:
    _check(
        isinstance(tensor, torch.Tensor)
        and tensor.is_cuda
        and tensor.dtype == torch.float32
        and tensor.is_contiguous(),
        f"{what}: expected a contiguous gfx950 float32 tensor",
    )


def _i64(tensor, what: str) -> None:
    _check(
        isinstance(tensor, torch.Tensor)
        and tensor.is_cuda
        and tensor.dtype == torch.int64
        and tensor.is_contiguous(),
        f"{what} must be a contiguous gfx950 int64 tensor",
    )


def _offsets(tensor, what: str) -> int:
    _i64(tensor, what)
    _check(tensor.dim() == 1 and tensor.numel() >= 1, f"{what} must be a one-dimensional exclusive prefix sum")
    return int(tensor.numel()) - 1


def _order(order, edges: int, what: str) -> None:
    if order is None:
        return
    _i64(order, f"{what} order")
    _check(order.dim() == 1 and order.numel() == edges, f"{what} order must have shape (n_edges,)")


def _same_device(reference: torch.Tensor, *others) -> None:
    for other in others:
        if other is not None:
            _check(other.device == reference.device, "all tensors must share a device")


def _ptr(tensor):
    return None if tensor is None or tensor.numel() == 0 else tensor.data_ptr()


# The raw handle of a device's current stream, without building a
# torch.cuda.Stream object per launch (the public call is the fallback).
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _current_stream(index: int) -> int:
    if _raw_stream is not None:
        return _raw_stream(index)
    return torch.cuda.current_stream(index).cuda_stream


class _on:
    """Make `device` current for the launch (the reference's CUDAGuard); yields its current stream."""

    __slots__ = ("index", "previous")

    def __init__(self, device: torch.device):
        current = torch.cuda.current_device()
        self.index = current if device.index is None else device.index
        self.previous = current

    def __enter__(self) -> int:
        if self.index != self.previous:
            torch.cuda.set_device(self.index)
        return _current_stream(self.index)

    def __exit__(self, *exc) -> None:
        if self.index != self.previous:
            torch.cuda.set_device(self.previous)


def _workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


# ---------------------------------------------------------------------------
# CSR construction (python/kernels/segment.py:46-71)
# ---------------------------------------------------------------------------

def segment_offsets(keys: torch.Tensor, n_nodes: int) -> torch.Tensor:
    """``[0] ++ cumsum(bincount(keys, minlength=n_nodes))``; ValueError on out-of-range keys."""
    _i64(keys, "segment offsets keys")
    _check(keys.dim() == 1, "segment offsets keys must be one-dimensional")
    n_nodes = int(n_nodes)
    offsets = torch.empty(n_nodes + 1, dtype=torch.int64, device=keys.device)
    nbytes = _LIB.dpa4k_segment_offsets_workspace_size(keys.numel(), n_nodes)
    workspace = _workspace(nbytes, keys.device)
    with _on(keys.device) as stream:
        status = _LIB.dpa4k_segment_offsets(
            _ptr(keys), keys.numel(), n_nodes, offsets.data_ptr(), workspace.data_ptr(), nbytes, stream
        )
    _lib.check(status, index_error=True)
    return offsets


def group_by_key(keys: torch.Tensor, n_nodes: int) -> tuple[torch.Tensor, torch.Tensor]:
    """``(stable argsort(keys), segment_offsets(keys))``; ValueError on out-of-range keys."""
    _i64(keys, "group_by_source keys")
    _check(keys.dim() == 1, "group_by_source keys must be one-dimensional")
    n_nodes = int(n_nodes)
    edges = keys.numel()
    order = torch.empty(edges, dtype=torch.int64, device=keys.device)
    offsets = torch.empty(n_nodes + 1, dtype=torch.int64, device=keys.device)
    nbytes = _LIB.dpa4k_group_by_key_workspace_size(edges, n_nodes)
    workspace = _workspace(nbytes, keys.device)
    with _on(keys.device) as stream:
        status = _LIB.dpa4k_group_by_key(
            _ptr(keys), edges, n_nodes, _ptr(order), offsets.data_ptr(), workspace.data_ptr(), nbytes, stream
        )
    _lib.check(status, index_error=True)
    return order, offsets


def group_by_key_async(keys: torch.Tensor, n_nodes: int, *, order=None, offsets=None, status=None,
                       workspace=None) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """``group_by_key`` without the host synchronisation: ``(order, offsets, status)``.

    ``status`` (a one-element int32 device tensor) receives bit 1 when a key is
    out of range (``order`` and ``offsets`` are then unspecified) and bit 2 when
    the keys were not already sorted; read it before trusting the result.  Any
    buffer passed in is used as is (``workspace`` of at least
    ``dpa4k_group_by_key_workspace_size`` bytes), so a caller that passes all of
    them allocates nothing and may capture the call in a HIP graph.
    """
    _i64(keys, "group_by_source keys")
    _check(keys.dim() == 1, "group_by_source keys must be one-dimensional")
    n_nodes = int(n_nodes)
    edges = keys.numel()
    order = torch.empty(edges, dtype=torch.int64, device=keys.device) if order is None else order
    offsets = torch.empty(n_nodes + 1, dtype=torch.int64, device=keys.device) if offsets is None else offsets
    status = torch.empty(1, dtype=torch.int32, device=keys.device) if status is None else status
    _i64(order, "group_by_source order")
    _i64(offsets, "group_by_source offsets")
    _check(order.numel() == edges and offsets.numel() == n_nodes + 1, "group_by_source output buffers have the wrong size")
    _check(status.is_cuda and status.dtype == torch.int32 and status.numel() >= 1, "status must be a gfx950 int32 tensor")
    nbytes = _LIB.dpa4k_group_by_key_workspace_size(edges, n_nodes)
    workspace = _workspace(nbytes, keys.device) if workspace is None else workspace
    _check(workspace.is_cuda and workspace.numel() * workspace.element_size() >= nbytes, "workspace is too small")
    with _on(keys.device) as stream:
        code = _LIB.dpa4k_group_by_key_async(
            _ptr(keys), edges, n_nodes, _ptr(order), offsets.data_ptr(), status.data_ptr(), workspace.data_ptr(),
            workspace.numel() * workspace.element_size(), stream,
        )
    _lib.check(code)
    return order, offsets, status


# ---------------------------------------------------------------------------
# segment_sum (csrc/segment_sum.cpp:214, :271)
# ---------------------------------------------------------------------------

def _segment_sum_checks(src, offsets, edge_scale, node_scale, order):
    _f32(src, "segment sum src")
    _check(src.dim() == 2, "segment sum src must have shape (n_edges, channels)")
    edges, channels = int(src.shape[0]), int(src.shape[1])
    _check(channels > 0, "segment sum requires at least one channel")
    nodes = _offsets(offsets, "segment sum offsets")
    if edge_scale is not None:
        _f32(edge_scale, "segment sum edge_scale")
        _check(edge_scale.dim() == 1 and edge_scale.numel() == edges,
               "segment sum edge_scale must have shape (n_edges,)")
    if node_scale is not None:
        _f32(node_scale, "segment sum node_scale")
        _check(node_scale.numel() == nodes, "segment sum node_scale must have one value per segment")
    _order(order, edges, "segment sum")
    _same_device(src, offsets, edge_scale, node_scale, order)
    return edges, nodes, channels


def segment_sum_forward(src, offsets, edge_scale=None, node_scale=None, order=None):
    edges, nodes, channels = _segment_sum_checks(src, offsets, edge_scale, node_scale, order)
    out = torch.empty((nodes, channels), dtype=torch.float32, device=src.device)
    if nodes == 0:
        return out
    with _on(src.device) as stream:
        status = _LIB.dpa4k_segment_sum_forward(
            _ptr(src), offsets.data_ptr(), _ptr(edge_scale), _ptr(node_scale), _ptr(order),
            out.data_ptr(), edges, nodes, channels, stream,
        )
    _lib.check(status)
    return out


def segment_sum_backward(grad_out, src, dst, offsets, edge_scale=None, node_scale=None,
                         want_node_scale_grad=False, order=None, *, want_edge_scale_grad=False):
    edges, nodes, channels = _segment_sum_checks(src, offsets, edge_scale, node_scale, order)
    _f32(grad_out, "segment sum grad_out")
    _check(grad_out.dim() == 2 and tuple(grad_out.shape) == (nodes, channels),
           "segment sum grad_out must have shape (n_nodes, channels)")
    _i64(dst, "segment sum dst")
    _check(dst.dim() == 1 and dst.numel() == edges, f"segment sum dst must have shape ({edges},)")
    _same_device(src, grad_out, dst)
    grad_src = torch.empty_like(src)
    node_grad = want_node_scale_grad and node_scale is not None
    edge_grad = want_edge_scale_grad and edge_scale is not None
    grad_node_scale = torch.empty_like(node_scale) if node_grad else None
    grad_edge_scale = torch.empty_like(edge_scale) if edge_grad else None
    if nodes > 0 and (edges > 0 or node_grad):
        with _on(src.device) as stream:
            status = _LIB.dpa4k_segment_sum_backward(
                grad_out.data_ptr(), _ptr(src), offsets.data_ptr(), _ptr(edge_scale),
                _ptr(node_scale), _ptr(order), _ptr(grad_src), _ptr(grad_edge_scale),
                None if grad_node_scale is None else grad_node_scale.data_ptr(),
                edges, nodes, channels, stream,
            )
        _lib.check(status)
    if want_edge_scale_grad:
        return grad_src, grad_node_scale, grad_edge_scale
    return grad_src, grad_node_scale


# ---------------------------------------------------------------------------
# segment_softmax (csrc/segment_softmax.cpp:235, :279)
# ---------------------------------------------------------------------------

def _softmax_checks(logit, env, offsets, order):
    _f32(logit, "segment softmax logit")
    _f32(env, "segment softmax env")
    _check(logit.dim() == 2, "segment softmax logit must have shape (n_edges, channels)")
    edges, channels = int(logit.shape[0]), int(logit.shape[1])
    _check(channels > 0, "segment softmax requires at least one channel")
    _check(env.dim() == 1 and env.numel() == edges, "segment softmax env must have shape (n_edges,)")
    nodes = _offsets(offsets, "segment softmax offsets")
    _order(order, edges, "segment softmax")
    _same_device(logit, env, offsets, order)
    return edges, nodes, channels


def _null_checks(tensor, nodes, channels, what):
    if tensor is None:
        return
    _f32(tensor, what)
    _check(tensor.numel() == nodes * channels, f"{what} must have shape (n_nodes, channels)")


class _TensorStamp:
    """Which tensor a plan was built from: the object itself (weakly held), its storage, size and version.

    A plan describes the values of its graph tensors when it was built.
    :meth:`matches` holds for that same object only, unchanged since: not
    for a copy, and not for a new tensor that the caching allocator placed
    at a freed tensor's address (the weak reference of a freed tensor is
    dead), nor after an in-place write (the version counter moves; an
    inference tensor has none, and is trusted while it lives).
    """

    __slots__ = ("ref", "stamp")

    def __init__(self, tensor: torch.Tensor):
        self.ref = weakref.ref(tensor)
        self.stamp = self._stamp_of(tensor)

    @staticmethod
    def _stamp_of(tensor: torch.Tensor):
        version = None if tensor.is_inference() else tensor._version
        return (tensor.data_ptr(), tensor.numel(), version)

    def matches(self, tensor: torch.Tensor) -> bool:
        return self.ref() is tensor and self.stamp == self._stamp_of(tensor)


def _offsets_fingerprint(offsets: torch.Tensor) -> _TensorStamp:
    return _TensorStamp(offsets)


class SoftmaxPlan:
    """Degree plan of one CSR (the long segments of ``offsets``) for one channel count.

    ``fingerprint`` identifies the ``offsets`` tensor the plan was built from:
    a plan only lists that CSR's long segments, and the kernels would leave
    any other long segment unwritten, so a plan is refused for any other
    tensor (a copy, or a new tensor at a freed one's address) and after an
    in-place write (:class:`_TensorStamp`).
    """

    __slots__ = ("words", "n_long", "capacity", "n_edges", "channels", "fingerprint")

    def __init__(self, words: torch.Tensor, n_long: int, capacity: int, n_edges: int, channels: int,
                 fingerprint=None):
        self.words, self.n_long, self.capacity = words, n_long, capacity
        self.n_edges, self.channels, self.fingerprint = n_edges, channels, fingerprint


def segment_softmax_plan(offsets, n_edges: int, channels: int) -> SoftmaxPlan:
    """Build the degree plan of ``offsets`` on its device (synchronises once)."""
    nodes = _offsets(offsets, "segment softmax offsets")
    _check(int(channels) > 0, "segment softmax requires at least one channel")
    nbytes = _LIB.dpa4k_segment_softmax_plan_size(nodes)
    words = torch.empty((max(int(nbytes), 8) + 7) // 8, dtype=torch.int64, device=offsets.device)
    n_long, capacity = _lib.ctypes.c_int64(0), _lib.ctypes.c_int64(0)
    with _on(offsets.device) as stream:
        status = _LIB.dpa4k_segment_softmax_plan(
            offsets.data_ptr(), int(n_edges), nodes, int(channels), words.data_ptr(), words.numel() * 8,
            _lib.ctypes.byref(n_long), _lib.ctypes.byref(capacity), stream,
        )
    _lib.check(status)
    return SoftmaxPlan(words, int(n_long.value), int(capacity.value), int(n_edges), int(channels),
                       _offsets_fingerprint(offsets))


def _plan_args(plan, offsets, edges, channels):
    if plan is None:
        return None
    _check(isinstance(plan, SoftmaxPlan) and plan.words.device == offsets.device
           and plan.n_edges == edges and plan.channels == channels
           and plan.fingerprint is not None and plan.fingerprint.matches(offsets),
           "segment softmax plan was built for another graph, device or channel count")
    return plan


def segment_softmax_forward(logit, env, offsets, null_logit=None, order=None, *, plan=None):
    edges, nodes, channels = _softmax_checks(logit, env, offsets, order)
    _null_checks(null_logit, nodes, channels, "segment softmax null_logit")
    _same_device(logit, null_logit)
    plan = _plan_args(plan, offsets, edges, channels)
    alpha = torch.empty((edges, channels), dtype=torch.float32, device=logit.device)
    null_alpha = None
    if null_logit is not None:
        null_alpha = torch.empty((nodes, channels), dtype=torch.float32, device=logit.device)
    if nodes == 0:
        return alpha, null_alpha
    with _on(logit.device) as stream:
        if plan is None:
            status = _LIB.dpa4k_segment_softmax_forward(
                _ptr(logit), _ptr(env), offsets.data_ptr(), _ptr(null_logit), _ptr(order), _ptr(alpha),
                _ptr(null_alpha), edges, nodes, channels, stream,
            )
        else:
            status = _LIB.dpa4k_segment_softmax_forward_planned(
                _ptr(logit), _ptr(env), offsets.data_ptr(), _ptr(null_logit), _ptr(order), _ptr(alpha),
                _ptr(null_alpha), edges, nodes, channels, plan.words.data_ptr(), plan.n_long, plan.capacity, stream,
            )
    _lib.check(status)
    return alpha, null_alpha


def segment_softmax_backward(alpha, grad_alpha, env, offsets, null_alpha=None,
                             grad_null_alpha=None, order=None, *, plan=None):
    edges, nodes, channels = _softmax_checks(alpha, env, offsets, order)
    plan = _plan_args(plan, offsets, edges, channels)
    _f32(grad_alpha, "segment softmax grad_alpha")
    _check(tuple(grad_alpha.shape) == tuple(alpha.shape), "segment softmax grad_alpha must match alpha")
    _same_device(alpha, grad_alpha)
    has_null = null_alpha is not None
    _check(has_null == (grad_null_alpha is not None),
           "segment softmax requires null_alpha and grad_null_alpha together")
    _null_checks(null_alpha, nodes, channels, "segment softmax null_alpha")
    _null_checks(grad_null_alpha, nodes, channels, "segment softmax grad_null_alpha")
    _same_device(alpha, null_alpha, grad_null_alpha)
    grad_logit = torch.empty_like(alpha)
    grad_null = torch.empty((nodes, channels), dtype=torch.float32, device=alpha.device) if has_null else None
    grad_env = torch.empty((edges,), dtype=torch.float32, device=alpha.device)
    if nodes == 0:
        return grad_logit, grad_null, grad_env
    with _on(alpha.device) as stream:
        if plan is None:
            status = _LIB.dpa4k_segment_softmax_backward(
                _ptr(alpha), _ptr(grad_alpha), _ptr(env), offsets.data_ptr(), _ptr(null_alpha),
                _ptr(grad_null_alpha), _ptr(order), _ptr(grad_logit), _ptr(grad_null), _ptr(grad_env),
                edges, nodes, channels, stream,
            )
        else:
            status = _LIB.dpa4k_segment_softmax_backward_planned(
                _ptr(alpha), _ptr(grad_alpha), _ptr(env), offsets.data_ptr(), _ptr(null_alpha),
                _ptr(grad_null_alpha), _ptr(order), _ptr(grad_logit), _ptr(grad_null), _ptr(grad_env),
                edges, nodes, channels, plan.words.data_ptr(), plan.n_long, plan.capacity, stream,
            )
    _lib.check(status)
    return grad_logit, grad_null, grad_env


# ---------------------------------------------------------------------------
# force_assembly (csrc/force_assembly.cpp:106)
# ---------------------------------------------------------------------------

class ForcePlan:
    """Blob layout of one graph for the planned force assembly.

    Built once per graph by :func:`force_assembly_plan`.  ``records`` is the
    buffer the planned kernels write on every call (per-piece destination
    sums and per-record source sums), so calls that share a plan must not
    overlap (one stream at a time).  ``fingerprint`` identifies the offsets
    and ``src_order`` tensors the plan describes; a plan is refused for any
    other tensor, even one at a freed tensor's address, and after an
    in-place write (:class:`_TensorStamp`).
    """

    __slots__ = ("plan", "records", "n_edges", "n_nodes", "value_bytes", "n_records", "n_pieces", "fingerprint")

    def __init__(self, plan: torch.Tensor, records: torch.Tensor, n_edges: int, n_nodes: int, value_bytes: int,
                 n_records: int, n_pieces: int, fingerprint):
        self.plan, self.records = plan, records
        self.n_edges, self.n_nodes, self.value_bytes = n_edges, n_nodes, value_bytes
        self.n_records, self.n_pieces, self.fingerprint = n_records, n_pieces, fingerprint


def _force_fingerprint(dst_offsets, src_offsets, src_order) -> tuple:
    return tuple(_TensorStamp(t) for t in (dst_offsets, src_offsets, src_order))


def _force_plan_matches(plan, dst_offsets, src_offsets, src_order) -> bool:
    return all(stamp.matches(t) for stamp, t in zip(plan.fingerprint, (dst_offsets, src_offsets, src_order)))


def force_assembly_plan(dst_offsets, src_offsets, src_order, edge_vec=None, *, value_bytes: int = 4) -> ForcePlan:
    """Blob plan of a graph for float32 (value_bytes 4) or float64 (8) values; synchronises the device.

    ``edge_vec`` is a geometry hint: atom positions are recovered from it
    along a breadth-first tree to order the atoms in space (``None`` keeps
    the natural order).  Results do not depend on it, only the speed does.
    """
    nodes = _offsets(dst_offsets, "force assembly dst_offsets")
    _check(_offsets(src_offsets, "force assembly src_offsets") == nodes,
           "force assembly offsets must describe the same atom count")
    _i64(src_order, "force assembly src_order")
    _check(src_order.dim() == 1, "force assembly src_order must be one-dimensional")
    _check(nodes > 0, "force assembly requires at least one atom")
    _check(value_bytes in (4, 8), "force assembly plan: value_bytes must be 4 or 8")
    _same_device(dst_offsets, src_offsets, src_order)
    edges = int(src_order.numel())
    hint = 0
    if edge_vec is not None:
        _check(isinstance(edge_vec, torch.Tensor) and edge_vec.is_contiguous() and edge_vec.dim() == 2
               and tuple(edge_vec.shape) == (edges, 3) and edge_vec.element_size() == value_bytes
               and edge_vec.dtype in (torch.float32, torch.float64),
               "force assembly plan: edge_vec must be a contiguous (n_edges, 3) tensor of the plan's dtype")
        _same_device(src_order, edge_vec)
        hint = edge_vec.data_ptr()
    nbytes = int(_LIB.dpa4k_force_assembly_plan_size(edges, nodes, value_bytes))
    plan = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=src_order.device)
    scratch_bytes = int(_LIB.dpa4k_force_assembly_plan_workspace_size(edges, nodes))
    workspace = _workspace(scratch_bytes, src_order.device)
    counts = (_lib.ctypes.c_int64 * 2)()
    with _on(src_order.device) as stream:
        status = _LIB.dpa4k_force_assembly_plan(
            dst_offsets.data_ptr(), src_offsets.data_ptr(), _ptr(src_order), hint, edges, nodes, value_bytes,
            plan.data_ptr(), nbytes, workspace.data_ptr(), scratch_bytes, counts, stream,
        )
    _lib.check(status, index_error=True)  # offsets that are not CSRs of the edge list: ValueError
    n_records, n_pieces = int(counts[0]), int(counts[1])
    records_bytes = int(_LIB.dpa4k_force_assembly_records_size(n_records, n_pieces, value_bytes))
    records = torch.empty(max(records_bytes, 1), dtype=torch.uint8, device=src_order.device)
    return ForcePlan(plan, records, edges, nodes, value_bytes, n_records, n_pieces,
                     _force_fingerprint(dst_offsets, src_offsets, src_order))


def force_assembly(grad_edge, edge_vec, dst_offsets, src_offsets, src_order, *, plan=None):
    """``(force, virial)``; with a :class:`ForcePlan` of this graph the blob kernels run."""
    for name, tensor in (("grad_edge", grad_edge), ("edge_vec", edge_vec)):
        _check(isinstance(tensor, torch.Tensor) and tensor.is_cuda and tensor.is_contiguous()
               and tensor.dtype in (torch.float32, torch.float64),
               f"force assembly {name}: expected a contiguous gfx950 float32 or float64 tensor")
    _check(grad_edge.dtype == edge_vec.dtype, "force assembly grad_edge and edge_vec must share a dtype")
    _check(grad_edge.dim() == 2 and grad_edge.shape[1] == 3, "force assembly grad_edge must have shape (n_edges, 3)")
    _check(tuple(edge_vec.shape) == tuple(grad_edge.shape), "force assembly edge_vec must match grad_edge")
    edges = int(grad_edge.shape[0])
    nodes = _offsets(dst_offsets, "force assembly dst_offsets")
    _check(_offsets(src_offsets, "force assembly src_offsets") == nodes,
           "force assembly offsets must describe the same atom count")
    _i64(src_order, "force assembly src_order")
    _check(src_order.dim() == 1 and src_order.numel() == edges, "force assembly src_order must have shape (n_edges,)")
    _check(nodes > 0, "force assembly requires at least one atom")
    _same_device(grad_edge, edge_vec, dst_offsets, src_offsets, src_order)
    force = torch.empty((nodes, 3), dtype=grad_edge.dtype, device=grad_edge.device)
    virial = torch.empty((nodes, 9), dtype=grad_edge.dtype, device=grad_edge.device)
    single = grad_edge.dtype == torch.float32
    if plan is not None:
        _check(isinstance(plan, ForcePlan) and plan.n_edges == edges and plan.n_nodes == nodes
               and plan.plan.device == grad_edge.device and plan.value_bytes == grad_edge.element_size()
               and _force_plan_matches(plan, dst_offsets, src_offsets, src_order),
               "force assembly plan was built for another graph, device or dtype")
        entry = _LIB.dpa4k_force_assembly_f32_planned if single else _LIB.dpa4k_force_assembly_f64_planned
        with _on(grad_edge.device) as stream:
            status = entry(_ptr(grad_edge), _ptr(edge_vec), force.data_ptr(), virial.data_ptr(), edges, nodes,
                           plan.plan.data_ptr(), plan.plan.numel(), plan.records.data_ptr(), plan.records.numel(),
                           plan.n_records, plan.n_pieces, None, stream)
        _lib.check(status)
        return force, virial
    entry = _LIB.dpa4k_force_assembly_f32 if single else _LIB.dpa4k_force_assembly_f64
    with _on(grad_edge.device) as stream:
        status = entry(_ptr(grad_edge), _ptr(edge_vec), dst_offsets.data_ptr(), src_offsets.data_ptr(),
                       _ptr(src_order), force.data_ptr(), virial.data_ptr(), edges, nodes, stream)
    _lib.check(status)
    return force, virial


# ---------------------------------------------------------------------------
# GIE zonal scatter (csrc/gie.cpp:148, :178)
# ---------------------------------------------------------------------------

def _gie_checks(zonal, radial, dst, radial_slot, inv_sqrt_deg):
    _f32(zonal, "GIE zonal")
    _f32(radial, "GIE radial")
    _f32(inv_sqrt_deg, "GIE inv_sqrt_deg")
    _check(zonal.dim() == 2, "GIE zonal must have shape (n_edges, n_rows)")
    _check(radial.dim() == 3, "GIE radial must have shape (n_edges, n_radial, channels)")
    edges, rows = int(zonal.shape[0]), int(zonal.shape[1])
    _check(radial.shape[0] == edges, "GIE radial edge dimension must match zonal")
    _i64(dst, "GIE dst")
    _check(dst.dim() == 1 and dst.numel() == edges, f"GIE dst must have shape ({edges},)")
    _i64(radial_slot, "GIE radial_slot")
    _check(radial_slot.dim() == 1 and radial_slot.numel() == rows, f"GIE radial_slot must have shape ({rows},)")
    _check(inv_sqrt_deg.dim() in (1, 3), "GIE inv_sqrt_deg must have shape (n_nodes,) or (n_nodes, 1, 1)")
    _check(inv_sqrt_deg.dim() != 3 or tuple(inv_sqrt_deg.shape[1:]) == (1, 1),
           "GIE inv_sqrt_deg must have shape (n_nodes, 1, 1)")
    _check(rows == 0 or radial.shape[1] > 0, "GIE radial slots are required for non-scalar rows")
    _check(edges == 0 or inv_sqrt_deg.shape[0] > 0, "GIE edges require destination nodes")
    _same_device(zonal, radial, dst, radial_slot, inv_sqrt_deg)
    return edges, rows, int(radial.shape[1]), int(radial.shape[2]), int(inv_sqrt_deg.shape[0])


def gie_group(dst, radial_slot, n_nodes: int, n_radial: int):
    """Destination CSR of an unsorted ``dst``: ``(offsets, order or None, info)``.

    ``order`` is None when ``dst`` is already non-decreasing; ``info`` bit 2
    says every radial slot feeds at most one row and bits 16..23 hold the most
    rows that read one slot.  The GIE kernels below take ``info`` as
    ``slot_info`` to pick their layout.  ValueError on out-of-range ``dst`` or
    ``radial_slot`` values.
    """
    edges, rows = int(dst.numel()), int(radial_slot.numel())
    offsets = torch.empty(n_nodes + 1, dtype=torch.int64, device=dst.device)
    order = torch.empty(max(edges, 1), dtype=torch.int64, device=dst.device)
    nbytes = _LIB.dpa4k_gie_group_workspace_size(edges, n_nodes)
    workspace = _workspace(nbytes, dst.device)
    info = _lib.ctypes.c_int32(0)
    with _on(dst.device) as stream:
        status = _LIB.dpa4k_gie_group(
            _ptr(dst), _ptr(radial_slot), edges, n_nodes, rows, n_radial, offsets.data_ptr(),
            order.data_ptr(), _lib.ctypes.byref(info), workspace.data_ptr(), nbytes, stream,
        )
    _lib.check(status, index_error=True)
    grouped = bool(info.value & 1)
    return offsets, (None if grouped else order[:edges]), int(info.value)


def gie_zonal_scatter_forward_csr(zonal, radial, offsets, order, radial_slot, inv_sqrt_deg, slot_info=0):
    edges, rows = int(zonal.shape[0]), int(zonal.shape[1])
    n_radial, channels = int(radial.shape[1]), int(radial.shape[2])
    nodes = int(inv_sqrt_deg.shape[0])
    out = torch.empty((nodes, rows + 1, channels), dtype=torch.float32, device=zonal.device)
    if nodes == 0 or channels == 0:
        return out.zero_()
    with _on(zonal.device) as stream:
        status = _LIB.dpa4k_gie_zonal_scatter_forward_csr(
            _ptr(zonal), _ptr(radial), offsets.data_ptr(), _ptr(order), _ptr(radial_slot),
            inv_sqrt_deg.data_ptr(), out.data_ptr(), edges, nodes, rows, n_radial, channels, int(slot_info), stream,
        )
    _lib.check(status)
    return out


def gie_rmsnorm_supported(n_rows: int, channels: int) -> bool:
    """Whether the fused GIE -> RMSNorm kernel takes rows of (n_rows + 1) * channels floats."""
    return bool(_LIB.dpa4k_gie_rmsnorm_supported(int(n_rows), int(channels)))


def gie_rmsnorm_forward_csr(zonal, radial, offsets, order, radial_slot, inv_sqrt_deg, scale, eps, keep_x=False):
    """Fused GIE zonal scatter and RMSNorm over each node's flattened (n_rows + 1) * channels row.

    Returns ``(y, x, inverse_rms)``: ``y`` shaped ``(n_nodes, n_rows + 1, channels)``, the pre-norm
    GIE output ``x`` of the same shape when ``keep_x`` (else None) and ``inverse_rms`` ``(n_nodes,)``.
    ``scale`` is a ``((n_rows + 1) * channels,)`` tensor or an empty one for no scale.
    """
    edges, rows = int(zonal.shape[0]), int(zonal.shape[1])
    n_radial, channels = int(radial.shape[1]), int(radial.shape[2])
    nodes = int(inv_sqrt_deg.shape[0])
    width = (rows + 1) * channels
    _check(gie_rmsnorm_supported(rows, channels),
           "GIE RMSNorm needs channels % 4 == 0 and rows of at most 2048 + channels floats")
    _f32(scale, "GIE RMSNorm scale")
    _check(scale.numel() in (0, width), f"GIE RMSNorm scale must have shape ({width},) or be empty")
    _same_device(zonal, radial, offsets, radial_slot, inv_sqrt_deg, scale)
    y = torch.empty((nodes, rows + 1, channels), dtype=torch.float32, device=zonal.device)
    x = torch.empty_like(y) if keep_x else None
    inverse_rms = torch.empty((nodes,), dtype=torch.float32, device=zonal.device)
    if nodes == 0:
        return y, x, inverse_rms
    with _on(zonal.device) as stream:
        status = _LIB.dpa4k_gie_rmsnorm_forward_csr(
            _ptr(zonal), _ptr(radial), offsets.data_ptr(), _ptr(order), _ptr(radial_slot), inv_sqrt_deg.data_ptr(),
            _ptr(scale), float(eps), y.data_ptr(), None if x is None else x.data_ptr(), inverse_rms.data_ptr(),
            edges, nodes, rows, n_radial, channels, stream,
        )
    _lib.check(status)
    return y, x, inverse_rms


def gie_zonal_scatter_backward_csr(grad_output, zonal, radial, offsets, order, radial_slot,
                                   inv_sqrt_deg, slot_info, *, need=(True, True, True)):
    edges, rows = int(zonal.shape[0]), int(zonal.shape[1])
    n_radial, channels = int(radial.shape[1]), int(radial.shape[2])
    nodes = int(inv_sqrt_deg.shape[0])
    grad_zonal = torch.empty_like(zonal) if need[0] else None
    grad_radial = torch.empty_like(radial) if need[1] else None
    grad_inv = torch.empty_like(inv_sqrt_deg) if need[2] else None
    if edges == 0 or rows == 0 or channels == 0 or nodes == 0:
        for tensor in (grad_zonal, grad_radial, grad_inv):
            if tensor is not None:
                tensor.zero_()
        return grad_zonal, grad_radial, grad_inv
    with _on(zonal.device) as stream:
        status = _LIB.dpa4k_gie_zonal_scatter_backward_csr(
            grad_output.data_ptr(), _ptr(zonal), _ptr(radial), offsets.data_ptr(), _ptr(order),
            _ptr(radial_slot), inv_sqrt_deg.data_ptr(), _ptr(grad_zonal), _ptr(grad_radial),
            _ptr(grad_inv), edges, nodes, rows, n_radial, channels, int(slot_info), stream,
        )
    _lib.check(status)
    return grad_zonal, grad_radial, grad_inv


def gie_zonal_scatter_forward(zonal, radial, dst, radial_slot, inv_sqrt_deg):
    edges, rows, n_radial, channels, nodes = _gie_checks(zonal, radial, dst, radial_slot, inv_sqrt_deg)
    if nodes == 0 or edges * rows * channels == 0:
        return torch.zeros((nodes, rows + 1, channels), dtype=torch.float32, device=zonal.device)
    offsets, order, info = gie_group(dst, radial_slot, nodes, n_radial)
    return gie_zonal_scatter_forward_csr(zonal, radial, offsets, order, radial_slot, inv_sqrt_deg, info)


def gie_zonal_scatter_backward(grad_output, zonal, radial, dst, radial_slot, inv_sqrt_deg):
    edges, rows, n_radial, channels, nodes = _gie_checks(zonal, radial, dst, radial_slot, inv_sqrt_deg)
    _f32(grad_output, "GIE grad_output")
    _same_device(zonal, grad_output)
    _check(grad_output.dim() == 3 and tuple(grad_output.shape) == (nodes, rows + 1, channels),
           "GIE grad_output must have shape (n_nodes, n_rows + 1, channels)")
    if nodes == 0 or edges * rows * channels == 0:
        return torch.zeros_like(zonal), torch.zeros_like(radial), torch.zeros_like(inv_sqrt_deg)
    offsets, order, info = gie_group(dst, radial_slot, nodes, n_radial)
    return gie_zonal_scatter_backward_csr(grad_output, zonal, radial, offsets, order, radial_slot,
                                          inv_sqrt_deg, info)


# ---------------------------------------------------------------------------
# RMSNorm (csrc/rmsnorm.cpp:99, :123)
# ---------------------------------------------------------------------------

def _rmsnorm_checks(x, scale):
    _f32(x, "RMSNorm input")
    _f32(scale, "RMSNorm scale")
    _same_device(x, scale)
    _check(x.dim() >= 1, "RMSNorm input must have at least one dimension")
    _check(x.shape[-1] > 0, "RMSNorm feature dimension must be positive")
    _check(scale.dim() == 1 and scale.numel() in (0, x.shape[-1]),
           "RMSNorm scale must be an empty vector or have shape (feature_dim,)")
    width = int(x.shape[-1])
    return x.numel() // width, width


def rmsnorm_forward(x, scale, eps):
    rows, width = _rmsnorm_checks(x, scale)
    eps = float(eps)
    _check(eps > 0.0 and eps != float("inf"), "RMSNorm eps must be a finite positive number")
    out = torch.empty_like(x)
    inverse_rms = torch.empty((rows,), dtype=torch.float32, device=x.device)
    if rows == 0:
        return out, inverse_rms
    with _on(x.device) as stream:
        status = _LIB.dpa4k_rmsnorm_forward(
            x.data_ptr(), _ptr(scale), out.data_ptr(), inverse_rms.data_ptr(), rows, width, eps, stream
        )
    _lib.check(status)
    return out, inverse_rms


def rmsnorm_backward(grad_output, x, scale, inverse_rms, compute_scale_grad):
    rows, width = _rmsnorm_checks(x, scale)
    _f32(grad_output, "RMSNorm grad_output")
    _f32(inverse_rms, "RMSNorm inverse_rms")
    _same_device(x, grad_output, inverse_rms)
    _check(tuple(grad_output.shape) == tuple(x.shape), "RMSNorm grad_output must have the input shape")
    _check(inverse_rms.dim() == 1 and inverse_rms.numel() == rows, "RMSNorm saved inverse_rms has an invalid shape")
    has_scale = scale.numel() != 0
    _check(not compute_scale_grad or has_scale, "cannot compute a scale gradient when scale is omitted")
    grad_x = torch.empty_like(x)
    grad_scale = (torch.empty((width,), dtype=torch.float32, device=x.device) if compute_scale_grad
                  else torch.empty((0,), dtype=torch.float32, device=x.device))
    nbytes = _LIB.dpa4k_rmsnorm_backward_workspace_size(rows, width) if compute_scale_grad else 0
    workspace = _workspace(nbytes, x.device) if compute_scale_grad else None
    with _on(x.device) as stream:
        status = _LIB.dpa4k_rmsnorm_backward(
            _ptr(grad_output), _ptr(x), _ptr(scale), _ptr(inverse_rms), _ptr(grad_x),
            grad_scale.data_ptr() if compute_scale_grad else None, rows, width,
            None if workspace is None else workspace.data_ptr(), nbytes, stream,
        )
    _lib.check(status)
    return grad_x, grad_scale


# ---------------------------------------------------------------------------
# edge-stream elementwise chain (no reference implementation: the fusion the
# reference designs as candidate C4, docs/task2-hip-fusion-plan.md:280-300)
# ---------------------------------------------------------------------------

EDGE_STREAM_ACTIVATIONS = {"none": 0, "silu": 1, "gate": 2}
EDGE_STREAM_MAX_TERMS = 4
EDGE_STREAM_MAX_GATE_ROWS = 64


def _edge_view(tensor, shape, what: str) -> torch.Tensor:
    """`tensor` broadcast to `shape` (zero strides on broadcast axes), checked as a gfx950 float32 operand."""
    _check(isinstance(tensor, torch.Tensor) and tensor.is_cuda and tensor.dtype == torch.float32,
           f"{what}: expected a gfx950 float32 tensor")
    try:
        return tensor.expand(shape)
    except RuntimeError as error:
        raise RuntimeError(f"{what} of shape {tuple(tensor.shape)} does not broadcast to {tuple(shape)}") from error


def _edge_operand(view: torch.Tensor) -> "_lib.EdgeOperand":
    return _lib.EdgeOperand(view.data_ptr(), (ctypes.c_int64 * 3)(*view.stride()))


def _byte_span(view: torch.Tensor) -> tuple[int, int]:
    """[first, last) bytes a view addresses (empty views address nothing)."""
    if view.numel() == 0:
        return view.data_ptr(), view.data_ptr()
    extent = 1 + sum((size - 1) * stride for size, stride in zip(view.shape, view.stride()))
    return view.data_ptr(), view.data_ptr() + 4 * extent


def edge_stream_combine(terms, shape, activation: str = "none", gate=None, gate_rows=None, out=None):
    """``act(sum_k (a_k * b_k) * coef_k)`` over (edge, row, channel) ``shape`` in one pass.

    ``terms``: 1 to 4 ``(coef, a, b)`` with ``b`` None for a factor of 1;
    ``a``, ``b`` and ``gate`` are float32 tensors that broadcast to ``shape``
    (``gate`` to ``(E, G, C)``).  ``activation``: "none", "silu" or "gate"
    (``gate_rows``: R ints, negative for the silu rows).  ``out`` may be
    given (contiguous, ``shape``) and may be the same memory as a contiguous
    full-shape operand; it must not overlap any other operand.
    """
    _check(isinstance(shape, (tuple, list, torch.Size)) and len(shape) == 3 and all(int(d) >= 0 for d in shape),
           "edge_stream_combine: shape must be (n_edges, n_rows, channels)")
    shape = tuple(int(d) for d in shape)
    edges, rows, channels = shape
    _check(1 <= len(terms) <= EDGE_STREAM_MAX_TERMS,
           f"edge_stream_combine takes 1 to {EDGE_STREAM_MAX_TERMS} terms, got {len(terms)}")
    _check(activation in EDGE_STREAM_ACTIVATIONS, f"edge_stream_combine: unknown activation {activation!r}")
    views = []
    for k, (coef, a, b) in enumerate(terms):
        views.append((float(coef), _edge_view(a, shape, f"edge_stream_combine term {k} a"),
                      None if b is None else _edge_view(b, shape, f"edge_stream_combine term {k} b")))
    device = views[0][1].device
    _same_device(views[0][1], *[v for _, a, b in views for v in (a, b)])
    gate_view, rows_array = None, None
    if activation == "gate":
        _check(gate_rows is not None and len(gate_rows) == rows,
               "edge_stream_combine: the gate activation needs one gate row per row")
        _check(rows <= EDGE_STREAM_MAX_GATE_ROWS,
               f"edge_stream_combine: the gate activation takes at most {EDGE_STREAM_MAX_GATE_ROWS} rows")
        rows_list = [int(g) for g in gate_rows]
        _check(all(g < EDGE_STREAM_MAX_GATE_ROWS for g in rows_list), "edge_stream_combine: gate row out of range")
        gates = max([g + 1 for g in rows_list if g >= 0], default=0)
        if gates > 0:
            _check(gate is not None, "edge_stream_combine: gated rows need a gate tensor")
            gate_view = _edge_view(gate, (edges, gates, channels), "edge_stream_combine gate")
            _same_device(views[0][1], gate_view)
        rows_array = (ctypes.c_int32 * max(rows, 1))(*rows_list)
    if out is None:
        out = torch.empty(shape, dtype=torch.float32, device=device)
    else:
        _f32(out, "edge_stream_combine out")
        _check(tuple(out.shape) == shape, f"edge_stream_combine: out must have shape {shape}")
        _same_device(views[0][1], out)
        out_span = _byte_span(out)
        operands = [v for _, a, b in views for v in (a, b) if v is not None] + ([gate_view] if gate_view is not None else [])
        for view in operands:
            if view.data_ptr() == out.data_ptr() and view.stride() == out.stride():
                continue  # the same elements: each is read before it is written, by the same thread
            first, last = _byte_span(view)
            _check(last <= out_span[0] or first >= out_span[1] or out.numel() == 0,
                   "edge_stream_combine: out overlaps an operand other than a full-shape alias")
    if out.numel() == 0:
        return out
    count = len(views)
    a_array = (_lib.EdgeOperand * count)(*[_edge_operand(a) for _, a, _ in views])
    b_array = (_lib.EdgeOperand * count)(*[_edge_operand(b) if b is not None else _lib.EdgeOperand()
                                           for _, _, b in views])
    coefs = (ctypes.c_float * count)(*[coef for coef, _, _ in views])
    gate_operand = _edge_operand(gate_view) if gate_view is not None else None
    with _on(device) as stream:
        status = _LIB.dpa4k_edge_stream_combine(
            a_array, b_array, coefs, count, EDGE_STREAM_ACTIVATIONS[activation],
            ctypes.byref(gate_operand) if gate_operand is not None else None, rows_array, out.data_ptr(),
            edges, rows, channels, stream,
        )
    _lib.check(status)
    return out


__all__ = [
    "force_assembly",
    "gie_zonal_scatter_backward",
    "gie_zonal_scatter_forward",
    "rmsnorm_backward",
    "rmsnorm_forward",
    "segment_softmax_backward",
    "segment_softmax_forward",
    "segment_sum_backward",
    "segment_sum_forward",
]
