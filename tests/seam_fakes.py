"""Stand-ins for DeepMD's SeZM seams, shared by the CPU and GPU seam tests.

They restate, from the reference's description of DeepMD's code
(docs/fused-operators.md:27-39,74-88; docs/deepmd-fused-dispatch.md:29-56 of
lipengfei1409/bysj), the two stock implementations the seams replace:

* ``stock_softmax`` -- ``segment_envelope_gated_softmax``: log-envelope gated
  softmax over each destination with a per-channel null logit
  ``log(softplus(z_bias) + eps)``;
* ``FakeBlock.forward_envelope`` -- ``zeros -> index_add_(dst, message *
  edge_env * gate) -> * inv_sqrt_deg``.

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
