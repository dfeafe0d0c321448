"""Vectorised float64 closed forms of the operators' gradients -- test infrastructure only.

The brute-force loops of ``oracle.loops`` are exact but O(E * C) Python
loops; the GPU parity tests need the same ground truth at thousands of edges.
These functions state each gradient's closed form with torch ops in float64,
independently of the autograd chains in ``oracle/``, so a GPU gradient can be
held to the fp32 rule against an fp64 truth.  Each one is pinned against the
exact loops in tests/test_oracle_pinning.py.

Closed forms (n = the segment of edge e):
  segment_softmax   S[n] = sum_e alpha ga + alpha0 ga0;  dlogit = alpha (ga - S[n]);
                    dnull = alpha0 (ga0 - S);  denv[e] = 2 / env[e] sum_c dlogit  (0 unless env > 0)
  segment_sum       dsrc = g[n] s[n] w[e];  dw[e] = sum_c g[n] s[n] src[e];  ds[n] = sum_c g[n] (sum_e w src)
  zonal_scatter     oracle.loops.zonal_scatter_backward_loop's formulas
  rmsnorm           u = g scale;  dx = inv u - x inv^3 mean(x u);  dscale = sum_rows g x inv
"""
from __future__ import annotations

import torch


def _d(tensor):
    return None if tensor is None else tensor.detach().cpu().double()


def segment_softmax_f64(logit, env, dst, n_nodes, null_logit=None):
    """alpha (and null alpha) in float64: the softmax of ``logit + 2 ln env`` over each segment."""
    logit, env, null = _d(logit), _d(env), _d(null_logit)
    dst = dst.detach().cpu()
    edges, channels = logit.shape
    valid = (env > 0).reshape(-1, 1)
    effective = torch.where(valid, logit + 2.0 * torch.log(env.clamp_min(1e-30)).reshape(-1, 1),
                            torch.full_like(logit, float("-inf")))
    peak = torch.full((n_nodes, channels), float("-inf"), dtype=torch.float64)
    if edges:
        peak.scatter_reduce_(0, dst.reshape(-1, 1).expand(edges, channels), effective, reduce="amax")
    if null is not None:
        peak = torch.maximum(peak, null)
    finite = torch.isfinite(peak)
    safe_peak = torch.where(finite, peak, torch.zeros_like(peak))
    weight = torch.where(valid & finite[dst], torch.exp(effective - safe_peak[dst]), torch.zeros_like(effective))
    null_weight = torch.exp(null - safe_peak) if null is not None else torch.zeros_like(peak)
    total = torch.zeros_like(peak).index_add_(0, dst, weight) + null_weight
    total = torch.where(total > 0, total, torch.ones_like(total))
    return weight / total[dst], (null_weight / total if null is not None else None)


def segment_softmax_backward_f64(grad_alpha, logit, env, dst, n_nodes, null_logit=None, grad_null_alpha=None):
    """``(grad_logit, grad_env, grad_null_logit)`` in float64 from the closed form."""
    alpha, null_alpha = segment_softmax_f64(logit, env, dst, n_nodes, null_logit)
    ga, env64 = _d(grad_alpha), _d(env)
    dst = dst.detach().cpu()
    expectation = torch.zeros((n_nodes, alpha.shape[1]), dtype=torch.float64).index_add_(0, dst, alpha * ga)
    grad_null = None
    if null_alpha is not None:
        gn = _d(grad_null_alpha) if grad_null_alpha is not None else torch.zeros_like(null_alpha)
        expectation = expectation + null_alpha * gn
        grad_null = null_alpha * (gn - expectation)
    grad_logit = alpha * (ga - expectation[dst])
    grad_env = torch.where(env64 > 0, grad_logit.sum(1) * 2.0 / torch.where(env64 > 0, env64, 1.0),
                           torch.zeros_like(env64))
    return grad_logit, grad_env, grad_null


def segment_sum_backward_f64(grad_out, src, dst, n_nodes, edge_scale=None, node_scale=None):
    """``(grad_src, grad_edge_scale, grad_node_scale)`` in float64 (None where a scale is absent)."""
    g, s64 = _d(grad_out), _d(src)
    dst = dst.detach().cpu()
    w = _d(edge_scale) if edge_scale is not None else torch.ones(s64.shape[0], dtype=torch.float64)
    s = _d(node_scale).reshape(-1) if node_scale is not None else torch.ones(n_nodes, dtype=torch.float64)
    scaled = g[dst] * s[dst].reshape(-1, 1)
    grad_src = scaled * w.reshape(-1, 1)
    grad_w = (scaled * s64).sum(1) if edge_scale is not None else None
    grad_s = None
    if node_scale is not None:
        prefix = torch.zeros_like(g).index_add_(0, dst, s64 * w.reshape(-1, 1))
        grad_s = (g * prefix).sum(1).reshape(node_scale.shape)
    return grad_src, grad_w, grad_s


def zonal_scatter_backward_f64(grad_output, zonal, radial, dst, radial_slot, inv_sqrt_deg):
    """``(grad_zonal, grad_radial, grad_inv_sqrt_deg)`` in float64; grad_inv has the inverse's shape."""
    g, z, rad = _d(grad_output), _d(zonal), _d(radial)
    dst, slots = dst.detach().cpu(), radial_slot.detach().cpu()
    inv = _d(inv_sqrt_deg).reshape(-1)
    edges, rows = z.shape
    gathered = rad[:, slots, :]  # [E, R, C]
    upstream = g[dst, 1:, :] * inv[dst].reshape(-1, 1, 1)  # inv[n] g[n, r+1, c]
    grad_zonal = (upstream * gathered).sum(2)
    grad_radial = torch.zeros_like(rad).index_add_(1, slots, upstream * z.reshape(edges, rows, 1))
    pre = torch.zeros((inv.shape[0], rows, rad.shape[2]), dtype=torch.float64).index_add_(
        0, dst, z.reshape(edges, rows, 1) * gathered)
    grad_inv = (g[:, 1:, :] * pre).sum((1, 2)).reshape(inv_sqrt_deg.shape)
    return grad_zonal, grad_radial, grad_inv


def rmsnorm_backward_f64(grad, x, scale=None, eps=1e-6):
    """``(grad_x, grad_scale or None)`` in float64 over the last axis."""
    g, xd = _d(grad), _d(x)
    width = xd.shape[-1]
    g2, x2 = g.reshape(-1, width), xd.reshape(-1, width)
    inv = 1.0 / torch.sqrt((x2 * x2).mean(1, keepdim=True) + eps)
    u = g2 * (_d(scale) if scale is not None else 1.0)
    grad_x = inv * u - x2 * inv ** 3 * (x2 * u).mean(1, keepdim=True)
    grad_scale = (g2 * x2 * inv).sum(0) if scale is not None else None
    return grad_x.reshape(xd.shape), grad_scale


def gie_rmsnorm_chain_f64(inputs, scale, up, eps):
    """Gradients of sum(up * y), y = rmsnorm(zonal_scatter(zonal, radial, dst, slot, inv)), in float64.

    Autograd through the two operators' formulas evaluated in float64 (the
    composition has no closed form worth restating).  Returns the gradients
    with respect to zonal, radial, inv_sqrt_deg (in its shape) and the scale
    (when given), and per node the sum of |d(loss)/d x * S| over the row (S the
    unnormalised scatter): the size of the terms that make up the inverse's
    gradient, which cancel because RMSNorm is scale invariant.
    """
    zonal, radial, dst, slots, inverse = (_d(t) if t.is_floating_point() else t.detach().cpu() for t in inputs)
    zonal, radial = zonal.requires_grad_(True), radial.requires_grad_(True)
    n_nodes, n_rows, channels = inverse.shape[0], zonal.shape[1], radial.shape[2]
    gathered = radial.gather(1, slots.reshape(1, -1, 1).expand(zonal.shape[0], n_rows, channels))
    summed = torch.zeros((n_nodes, n_rows + 1, channels), dtype=torch.float64)
    summed[:, 1:, :] = summed[:, 1:, :].index_add(0, dst, zonal.unsqueeze(-1) * gathered)
    inv = inverse.reshape(-1).clone().requires_grad_(True)
    x = (summed * inv.reshape(-1, 1, 1)).reshape(n_nodes, -1)
    x.retain_grad()
    y = x * torch.rsqrt(x.pow(2).mean(dim=1, keepdim=True) + eps)
    s = None if scale is None else _d(scale).requires_grad_(True)
    if s is not None:
        y = y * s
    (y * _d(up).reshape(n_nodes, -1)).sum().backward()
    terms = (x.grad * summed.detach().reshape(n_nodes, -1)).abs().sum(dim=1)
    grads = (zonal.grad, radial.grad, inv.grad.reshape(inverse.shape)) + (() if s is None else (s.grad,))
    return tuple(g.detach() for g in grads), terms.detach()
