"""CPU oracle of the segmented operators -- test infrastructure only.

Restates, with the same ATen op order:
  * python/kernels/segment.py:46-71   segment_offsets, group_by_source
  * python/reference/segment.py:14-36 CSR validation (bincount of dst == offsets)
  * python/reference/segment.py:39-60 segment_sum_reference
  * python/reference/segment.py:63-118 segment_softmax_reference
  * python/reference/segment.py:121-142 force_assembly_reference
of lipengfei1409/bysj.  The backward oracles are torch autograd through the
same chains.  ``force_assembly_reference`` also accepts float64 (the fp64
extension of the kernel); every other function is float32 like the reference.
"""
from __future__ import annotations

import torch


def segment_offsets(dst: torch.Tensor, n_nodes: int) -> torch.Tensor:
    """``[0] ++ cumsum(bincount(dst, minlength=n_nodes))`` (python/kernels/segment.py:46-57)."""
    if not isinstance(dst, torch.Tensor):
        raise TypeError("segment offsets require a tensor of destinations")
    if dst.dtype != torch.int64:
        raise TypeError("segment offsets require int64 destinations")
    if n_nodes <= 0:
        raise ValueError("segment offsets require a positive node count")
    if dst.numel() and (int(dst.min()) < 0 or int(dst.max()) >= n_nodes):
        raise ValueError("destination values must be within the node range")
    counts = torch.bincount(dst, minlength=n_nodes)
    return torch.cat([counts.new_zeros(1), counts.cumsum(0)])


def group_by_source(src: torch.Tensor, n_nodes: int) -> tuple[torch.Tensor, torch.Tensor]:
    """``(argsort(src, stable=True), segment_offsets(src))`` (python/kernels/segment.py:60-71)."""
    if not isinstance(src, torch.Tensor):
        raise TypeError("group_by_source requires a tensor of sources")
    if src.dtype != torch.int64:
        raise TypeError("group_by_source requires int64 sources")
    if n_nodes <= 0:
        raise ValueError("group_by_source requires a positive node count")
    if src.numel() and (int(src.min()) < 0 or int(src.max()) >= n_nodes):
        raise ValueError("source values must be within the node range")
    return torch.argsort(src, stable=True), segment_offsets(src, n_nodes)


def _node_count(offsets: torch.Tensor) -> int:
    if offsets.dim() != 1 or offsets.numel() < 2:
        raise ValueError("offsets must be a one-dimensional prefix sum of at least two entries")
    return int(offsets.numel()) - 1


def _check_grouping(dst: torch.Tensor, offsets: torch.Tensor, n_edges: int, name: str) -> None:
    """python/reference/segment.py:20-36: dst in range and offsets == its CSR."""
    if dst.dtype != torch.int64:
        raise TypeError(f"{name} dst must be int64")
    if dst.ndim != 1 or dst.shape[0] != n_edges:
        raise ValueError(f"{name} dst must have shape (n_edges,)")
    if offsets.dtype != torch.int64:
        raise TypeError(f"{name} offsets must be int64")
    n_nodes = _node_count(offsets)
    if dst.numel() and (int(dst.min()) < 0 or int(dst.max()) >= n_nodes):
        raise ValueError(f"{name} dst values must be within the node range")
    counts = torch.bincount(dst, minlength=n_nodes) if dst.numel() else dst.new_zeros(n_nodes)
    if not torch.equal(torch.cat([counts.new_zeros(1), counts.cumsum(0)]), offsets):
        raise ValueError("offsets must be the exclusive prefix sum of the dst group sizes")


def segment_sum_reference(src, dst, offsets, edge_scale=None, node_scale=None):
    """``out[n] = node_scale[n] * sum_{dst(e)=n} edge_scale[e] * src[e]``.

    Chain (python/reference/segment.py:54-60): ``src * edge_scale`` ->
    ``zeros`` -> ``index_add_(0, dst, .)`` -> ``* node_scale``.
    """
    if src.dtype != torch.float32:
        raise TypeError("segment sum src must be float32")
    if src.ndim != 2:
        raise ValueError("segment sum src must have shape (n_edges, channels)")
    n_nodes = _node_count(offsets)
    _check_grouping(dst, offsets, src.shape[0], "segment sum")
    if edge_scale is not None and (edge_scale.dtype != torch.float32 or edge_scale.shape != (src.shape[0],)):
        raise ValueError("segment sum edge_scale must be float32 with shape (n_edges,)")
    if node_scale is not None and (node_scale.dtype != torch.float32 or node_scale.numel() != n_nodes):
        raise ValueError("segment sum node_scale must be float32 with one value per segment")
    weighted = src if edge_scale is None else src * edge_scale.reshape(-1, 1)
    out = weighted.new_zeros((n_nodes, src.shape[1]))
    if weighted.numel():
        out.index_add_(0, dst, weighted)
    if node_scale is not None:
        out = out * node_scale.reshape(n_nodes, 1)
    return out


def segment_sum_backward_reference(grad_out, src, dst, offsets, edge_scale=None, node_scale=None):
    """Autograd of :func:`segment_sum_reference`: ``(grad_src, grad_edge_scale, grad_node_scale)``."""
    with torch.enable_grad():
        leaves = [src.detach().clone().requires_grad_(True)]
        scale_e = None if edge_scale is None else edge_scale.detach().clone().requires_grad_(True)
        scale_n = None if node_scale is None else node_scale.detach().clone().requires_grad_(True)
        inputs = leaves + [t for t in (scale_e, scale_n) if t is not None]
        out = segment_sum_reference(leaves[0], dst, offsets, scale_e, scale_n)
        grads = torch.autograd.grad(out, inputs, grad_out, allow_unused=True)
    grads = list(grads)
    grad_src = grads.pop(0)
    grad_e = grads.pop(0) if scale_e is not None else None
    grad_n = grads.pop(0) if scale_n is not None else None
    return grad_src, grad_e, grad_n


def segment_softmax_reference(logit, env, dst, offsets, null_logit=None):
    """Per-segment, per-channel softmax with the envelope folded into the logit.

    ``l_e = logit_e + 2 ln max(env_e, 1e-30)`` for ``env_e > 0`` (other edges
    excluded); ``m`` = max over the segment and the null logit; returns
    ``(alpha, null_alpha)`` with ``alpha = exp(l - m) / D``.  Chain of
    python/reference/segment.py:84-118.
    """
    if logit.dtype != torch.float32 or env.dtype != torch.float32:
        raise TypeError("segment softmax logit and env must be float32")
    if logit.ndim != 2 or env.shape != (logit.shape[0],):
        raise ValueError("segment softmax expects logit (n_edges, channels) and env (n_edges,)")
    n_edges, channels = logit.shape
    n_nodes = _node_count(offsets)
    _check_grouping(dst, offsets, n_edges, "segment softmax")
    if null_logit is not None and (null_logit.dtype != torch.float32 or null_logit.shape != (n_nodes, channels)):
        raise ValueError("segment softmax null_logit must be float32 (n_nodes, channels)")

    mask = (env > 0).reshape(-1, 1)
    log_env = 2.0 * torch.log(env.clamp_min(1e-30)).reshape(-1, 1)
    effective = torch.where(mask, logit + log_env, torch.full_like(logit, float("-inf")))

    peak = torch.full((n_nodes, channels), float("-inf"), dtype=logit.dtype)
    if n_edges:
        index = dst.reshape(-1, 1).expand(n_edges, channels).contiguous()
        peak.scatter_reduce_(0, index, effective, reduce="amax", include_self=True)
    if null_logit is not None:
        peak = torch.maximum(peak, null_logit)
    finite = peak > float("-inf")

    if n_edges:
        weights = torch.where(
            finite.index_select(0, dst), torch.exp(effective - peak.index_select(0, dst)), torch.zeros_like(effective)
        )
    else:
        weights = effective
    total = logit.new_zeros((n_nodes, channels))
    if n_edges:
        total.index_add_(0, dst, weights)
    if null_logit is not None:
        null_weight = torch.where(finite, torch.exp(null_logit - peak), torch.zeros_like(peak))
    else:
        null_weight = torch.zeros_like(total)
    total = total + null_weight
    safe = torch.where(total > 0, total, torch.ones_like(total))
    alpha = weights / safe.index_select(0, dst) if n_edges else weights
    null_alpha = null_weight / safe if null_logit is not None else None
    return alpha, null_alpha


def segment_softmax_backward_reference(grad_alpha, logit, env, dst, offsets, null_logit=None, grad_null_alpha=None):
    """Autograd of :func:`segment_softmax_reference`: ``(grad_logit, grad_env, grad_null_logit)``."""
    with torch.enable_grad():
        x = logit.detach().clone().requires_grad_(True)
        e = env.detach().clone().requires_grad_(True)
        n = None if null_logit is None else null_logit.detach().clone().requires_grad_(True)
        alpha, null_alpha = segment_softmax_reference(x, e, dst, offsets, n)
        outputs, cotangents, inputs = [alpha], [grad_alpha], [x, e]
        if n is not None:
            outputs.append(null_alpha)
            cotangents.append(grad_null_alpha if grad_null_alpha is not None else torch.zeros_like(null_alpha))
            inputs.append(n)
        grads = torch.autograd.grad(outputs, inputs, cotangents, allow_unused=True)
    grad_logit, grad_env = grads[0], grads[1]
    grad_null = grads[2] if n is not None else None
    if grad_env is None:
        grad_env = torch.zeros_like(env)
    return grad_logit, grad_env, grad_null


def force_assembly_reference(grad_edge, edge_vec, src, dst, dst_offsets, src_offsets):
    """``F_k = sum_{dst=k} g - sum_{src=k} g``, ``W_k = sum_{src=k} -(g outer v)``.

    Chain of python/reference/segment.py:134-142 (two ``index_add_`` plus the
    source-side outer product), in the dtype of the inputs (float32 like the
    reference, or float64 for the fp64 extension).
    """
    if grad_edge.dtype not in (torch.float32, torch.float64) or grad_edge.ndim != 2 or grad_edge.shape[1] != 3:
        raise ValueError("force assembly grad_edge must be float32/float64 (n_edges, 3)")
    if edge_vec.shape != grad_edge.shape or edge_vec.dtype != grad_edge.dtype:
        raise ValueError("force assembly edge_vec must match grad_edge")
    n_edges = grad_edge.shape[0]
    n_nodes = _node_count(dst_offsets)
    _check_grouping(dst, dst_offsets, n_edges, "force assembly destination")
    _check_grouping(src, src_offsets, n_edges, "force assembly source")
    if _node_count(src_offsets) != n_nodes:
        raise ValueError("force assembly offsets must describe the same atom count")
    force = grad_edge.new_zeros((n_nodes, 3))
    virial = grad_edge.new_zeros((n_nodes, 9))
    if n_edges:
        force.index_add_(0, dst, grad_edge)
        force.index_add_(0, src, -grad_edge)
        outer = -(grad_edge.unsqueeze(2) * edge_vec.unsqueeze(1)).reshape(n_edges, 9)
        virial.index_add_(0, src, outer)
    return force, virial


__all__ = [
    "force_assembly_reference",
    "group_by_source",
    "segment_offsets",
    "segment_softmax_backward_reference",
    "segment_softmax_reference",
    "segment_sum_backward_reference",
    "segment_sum_reference",
]
