"""Stand-ins for DeepMD's SeZM seams, shared by the CPU and GPU seam tests.

They restate, from the reference's description of DeepMD's code
(docs/fused-operators.md:27-39,74-88; docs/deepmd-fused-dispatch.md:29-56 of
lipengfei1409/bysj), the two stock implementations the seams replace:

* ``stock_softmax`` -- ``segment_envelope_gated_softmax``: log-envelope gated
  softmax over each destination with a per-channel null logit
  ``log(softplus(z_bias) + eps)``;
* ``FakeBlock.forward_envelope`` -- ``zeros -> index_add_(dst, message *
  edge_env * gate) -> * inv_sqrt_deg``.

* ``stock_edge_force_virial`` -- DeepMD's edge force/virial assembly for one
  frame, restated from the call the reference quotes
  (docs/fused-operators.md:111-133): CSR views from ``argsort`` +
  ``searchsorted``, two ``index_add_`` for the force, the source-side outer
  product ``-g (x) edge_vec`` scattered into the atom virial.  DeepMD's own
  ``edge_force_virial`` is not in this container, so the output layout
  (``force.reshape(-1)``, ``atom_virial.reshape(-1)``, a ``[1, 9]`` frame
  virial, an unused fourth value) is this stand-in's reading of the quote.

``OracleOps`` is an operator bundle that answers with the CPU oracle.
"""
from __future__ import annotations

import types

import torch

from oracle import segment as ref


def grouped_dst(counts, device="cpu"):
    counts_t = torch.tensor(counts, dtype=torch.int64)
    dst = torch.repeat_interleave(torch.arange(len(counts), dtype=torch.int64), counts_t)
    return dst.to(device)


def dst_from_csr(offsets, order):
    counts = (offsets[1:] - offsets[:-1]).cpu()
    grouped = torch.repeat_interleave(torch.arange(counts.numel(), dtype=torch.int64), counts).to(offsets.device)
    if order is None:
        return grouped
    dst = torch.empty_like(grouped)
    dst[order] = grouped
    return dst


class OracleOps:
    """Operator bundle computing with the oracle; records the calls it receives."""

    def __init__(self):
        self.calls = []

    def segment_softmax(self, logit, env, offsets, null_logit=None, *, order=None):
        self.calls.append(("softmax", tuple(logit.shape)))
        alpha, null_alpha = ref.segment_softmax_reference(logit, env, dst_from_csr(offsets, order), offsets, null_logit)
        return alpha if null_logit is None else (alpha, null_alpha)

    def segment_sum(self, src, dst, offsets, edge_scale=None, node_scale=None, *, order=None):
        self.calls.append(("sum", tuple(src.shape)))
        return ref.segment_sum_reference(src, dst_from_csr(offsets, order), offsets, edge_scale, node_scale)

    def force_assembly(self, grad_edge, edge_vec, src, dst, dst_offsets, src_offsets=None, src_order=None):
        """kernels.segment.force_assembly: ``src``/``dst`` may be None when the CSR views are given."""
        self.calls.append(("force", tuple(grad_edge.shape)))
        dst = dst_from_csr(dst_offsets, None) if dst is None else dst
        src = dst_from_csr(src_offsets, src_order) if src is None else src
        return ref.force_assembly_reference(grad_edge, edge_vec, src, dst, dst_offsets, src_offsets)


def edge_force_virial_call(g, edge_vec, dst_ext, src_ext, n_ext, *, edge_mask=None, frames=1, optional=None):
    """The argument list of DeepMD's call: CSR views from argsort + searchsorted (quoted chain)."""
    dst_order = torch.argsort(dst_ext)
    src_order = torch.argsort(src_ext)
    boundaries = torch.arange(n_ext + 1, device=g.device, dtype=dst_ext.dtype)
    dst_row_ptr = torch.searchsorted(dst_ext.index_select(0, dst_order), boundaries)
    src_row_ptr = torch.searchsorted(src_ext.index_select(0, src_order), boundaries)
    scatter_index = torch.zeros_like(dst_ext)
    mask = torch.ones(g.shape[0], dtype=torch.bool, device=g.device) if edge_mask is None else edge_mask
    empty = edge_vec.new_empty(0) if optional is None else optional
    return (g.contiguous(), edge_vec.contiguous(), scatter_index, mask, dst_order, dst_row_ptr, src_order,
            src_row_ptr, n_ext // frames, empty, n_ext, True)


def stock_edge_force_virial(g, edge_vec, edge_scatter_index, edge_mask, dst_order, dst_row_ptr, src_order,
                            src_row_ptr, n_node_per_frame, optional, n_ext, flag):
    """DeepMD's edge force/virial of one frame with torch scatters (masked edges contribute nothing)."""
    del edge_scatter_index, n_node_per_frame, optional, flag
    dst = dst_from_csr(dst_row_ptr, dst_order)
    src = dst_from_csr(src_row_ptr, src_order)
    kept = torch.where(edge_mask.reshape(-1, 1), g, torch.zeros_like(g))
    force = g.new_zeros((n_ext, 3)).index_add_(0, dst, kept).index_add_(0, src, -kept)
    outer = -(kept.unsqueeze(2) * edge_vec.unsqueeze(1)).reshape(-1, 9)
    atom_virial = g.new_zeros((n_ext, 9)).index_add_(0, src, outer)
    return force.reshape(-1), atom_virial.reshape(-1), atom_virial.sum(0, keepdim=True), None


def force_namespace(name="fake.pt_expt.kernels.edge_force_virial", attribute="edge_force_virial"):
    module = types.ModuleType(name)
    setattr(module, attribute, stock_edge_force_virial)
    return module


def stock_softmax(logits, edge_env, dst, n_nodes, z_bias_raw, eps, src_weight=None):
    """DeepMD's eager gated softmax (float32, any device), restated with torch scatter ops."""
    n_edges, n_focus, n_head = logits.shape
    channels = n_focus * n_head
    flat = logits.reshape(n_edges, channels)
    env = edge_env.reshape(n_edges, 1)
    log_weight = torch.where(env > 0, 2.0 * torch.log(env.clamp_min(1e-30)), torch.full_like(env, float("-inf")))
    effective = flat + log_weight
    null = torch.log(torch.nn.functional.softplus(z_bias_raw.reshape(-1)) + eps).reshape(1, channels)
    peak = null.expand(n_nodes, channels).clone()
    index = dst.reshape(-1, 1).expand(n_edges, channels)
    peak = peak.scatter_reduce(0, index, effective, reduce="amax", include_self=True)
    weights = torch.exp(effective - peak[dst])
    total = torch.exp(null - peak).index_add(0, dst, weights)
    return (weights / total[dst]).reshape(n_edges, n_focus, n_head)


def softmax_namespace(name="fake.sezm_nn.attention"):
    module = types.ModuleType(name)
    module.segment_envelope_gated_softmax = stock_softmax
    return module


class FakeEdgeCache:
    def __init__(self, counts, *, gate=False, device="cpu", seed=0):
        gen = torch.Generator().manual_seed(seed)
        self.dst = grouped_dst(counts, device)
        n_edges, n_nodes = int(self.dst.numel()), len(counts)
        self.edge_env = (torch.rand(n_edges, 1, generator=gen) + 0.1).to(device)
        self.inv_sqrt_deg = (torch.rand(n_nodes, 1, 1, generator=gen) + 0.5).to(device)
        self.edge_src_gate = (torch.rand(n_edges, 1, generator=gen) + 0.5).to(device) if gate else None


class FakeBlock:
    """An SO(2) block: ``edge_message`` plus the stock ``forward_envelope``."""

    def __init__(self, message):
        self.training = False
        self._segment_softmax_fn = None
        self.message = message

    def edge_message(self, x, edge_cache, radial_feat):
        return self.message, None

    def forward_envelope(self, x, edge_cache, radial_feat):
        message, _ = self.edge_message(x, edge_cache, radial_feat)
        weight = edge_cache.edge_env
        if edge_cache.edge_src_gate is not None:
            weight = weight * edge_cache.edge_src_gate
        out = x.new_zeros(x.shape)
        out = out.index_add(0, edge_cache.dst, message * weight.unsqueeze(-1))
        return out * edge_cache.inv_sqrt_deg


class FakeModel:
    def __init__(self, blocks):
        self.blocks = list(blocks)

    def modules(self):
        return iter(self.blocks)
