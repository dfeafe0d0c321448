"""Brute-force restatements used to pin the oracle -- test infrastructure only.

Each function recomputes an operator element by element with explicit
Python/numpy loops, independently of the vectorised ATen chains in
``oracle.segment`` / ``oracle.gie`` / ``oracle.rmsnorm``:

* ``*_loop`` functions work in float64 (``math.fsum`` where an exactly
  rounded sum is wanted) and serve as ground truth;
* ``segment_sum_sequential_f32`` accumulates in float32 in edge order, the
  arithmetic a sequential ``index_add_`` performs, so it must agree with the
  oracle (and with the sequential gfx950 kernels) bit for bit.

Inputs are numpy arrays (or anything ``np.asarray`` accepts).  Sizes should
stay small: these are O(E * C) Python loops.
"""
from __future__ import annotations

import math

import numpy as np


def _np(value, dtype=None):
    if value is None:
        return None
    if hasattr(value, "detach"):
        value = value.detach().cpu().numpy()
    return np.asarray(value, dtype=dtype)


def segment_sum_loop(src, dst, n_nodes, edge_scale=None, node_scale=None):
    """float64 ``out[n] = s[n] * sum_{dst(e)=n} w[e] * src[e]`` with exactly rounded sums."""
    src, dst = _np(src, np.float64), _np(dst, np.int64)
    w = _np(edge_scale, np.float64)
    s = _np(node_scale, np.float64)
    channels = src.shape[1]
    out = np.zeros((n_nodes, channels))
    for node in range(n_nodes):
        edges = np.nonzero(dst == node)[0]
        for c in range(channels):
            terms = [src[e, c] * (w[e] if w is not None else 1.0) for e in edges]
            out[node, c] = math.fsum(terms) * (s.reshape(-1)[node] if s is not None else 1.0)
    return out


def segment_sum_sequential_f32(src, dst, n_nodes, edge_scale=None, node_scale=None):
    """float32, edge-ordered accumulation: ``acc = acc + (src[e] * w[e])`` then ``* s``."""
    src, dst = _np(src, np.float32), _np(dst, np.int64)
    w = _np(edge_scale, np.float32)
    s = _np(node_scale, np.float32)
    out = np.zeros((n_nodes, src.shape[1]), dtype=np.float32)
    for e in range(src.shape[0]):
        term = src[e] * w[e] if w is not None else src[e]
        out[dst[e]] = out[dst[e]] + term.astype(np.float32)
    if s is not None:
        out = out * s.reshape(-1, 1)
    return out


def segment_softmax_loop(logit, env, dst, n_nodes, null_logit=None):
    """float64 per-segment softmax with the envelope in the logit; returns (alpha, null_alpha)."""
    logit, env, dst = _np(logit, np.float64), _np(env, np.float64), _np(dst, np.int64)
    null = _np(null_logit, np.float64)
    n_edges, channels = logit.shape
    alpha = np.zeros((n_edges, channels))
    null_alpha = np.zeros((n_nodes, channels)) if null is not None else None
    for node in range(n_nodes):
        edges = [e for e in range(n_edges) if dst[e] == node]
        for c in range(channels):
            values = {e: logit[e, c] + 2.0 * math.log(max(env[e], 1e-30)) for e in edges if env[e] > 0}
            candidates = list(values.values()) + ([null[node, c]] if null is not None else [])
            if not candidates:
                continue
            peak = max(candidates)
            weights = {e: math.exp(v - peak) for e, v in values.items()}
            null_weight = math.exp(null[node, c] - peak) if null is not None else 0.0
            total = math.fsum(list(weights.values()) + [null_weight])
            for e, weight in weights.items():
                alpha[e, c] = weight / total
            if null is not None:
                null_alpha[node, c] = null_weight / total
    return alpha, null_alpha


def force_assembly_loop(grad_edge, edge_vec, src, dst, n_nodes):
    """Exactly rounded (``math.fsum``) float64 force and virial."""
    g, v = _np(grad_edge, np.float64), _np(edge_vec, np.float64)
    src, dst = _np(src, np.int64), _np(dst, np.int64)
    force_terms = [[[] for _ in range(3)] for _ in range(n_nodes)]
    virial_terms = [[[] for _ in range(9)] for _ in range(n_nodes)]
    for e in range(g.shape[0]):
        for r in range(3):
            force_terms[dst[e]][r].append(g[e, r])
            force_terms[src[e]][r].append(-g[e, r])
            for c in range(3):
                virial_terms[src[e]][3 * r + c].append(-g[e, r] * v[e, c])
    force = np.array([[math.fsum(t) for t in row] for row in force_terms]).reshape(n_nodes, 3)
    virial = np.array([[math.fsum(t) for t in row] for row in virial_terms]).reshape(n_nodes, 9)
    return force, virial


def zonal_scatter_loop(zonal, radial, dst, radial_slot, inv_sqrt_deg):
    """float64 GIE scatter, normalised after the exactly rounded sum."""
    zonal, radial = _np(zonal, np.float64), _np(radial, np.float64)
    dst, slots = _np(dst, np.int64), _np(radial_slot, np.int64)
    inv = _np(inv_sqrt_deg, np.float64).reshape(-1)
    n_edges, n_rows = zonal.shape
    channels = radial.shape[2]
    out = np.zeros((inv.shape[0], n_rows + 1, channels))
    for node in range(inv.shape[0]):
        edges = np.nonzero(dst == node)[0]
        for r in range(n_rows):
            for c in range(channels):
                total = math.fsum(zonal[e, r] * radial[e, slots[r], c] for e in edges)
                out[node, r + 1, c] = total * inv[node]
    return out


def zonal_scatter_backward_loop(grad_output, zonal, radial, dst, radial_slot, inv_sqrt_deg):
    """float64 closed-form gradients of the GIE scatter, exactly rounded sums.

    With n = dst[e], g = grad_output and pre[n, r+1, c] = sum_{dst[e]=n} zonal[e, r] radial[e, slot[r], c]:
      grad_zonal[e, r]     = inv[n] * sum_c g[n, r+1, c] radial[e, slot[r], c]
      grad_radial[e, s, c] = sum_{r: slot[r] = s} inv[n] g[n, r+1, c] zonal[e, r]   (shared slots summed)
      grad_inv[n]          = sum_{r, c} g[n, r+1, c] pre[n, r+1, c]                  (row 0 of pre is zero)
    grad_inv takes the shape of ``inv_sqrt_deg``.
    """
    g = _np(grad_output, np.float64)
    zonal, radial = _np(zonal, np.float64), _np(radial, np.float64)
    dst, slots = _np(dst, np.int64), _np(radial_slot, np.int64)
    inv_shape = np.shape(_np(inv_sqrt_deg))
    inv = _np(inv_sqrt_deg, np.float64).reshape(-1)
    n_edges, n_rows = zonal.shape
    n_radial, channels = radial.shape[1], radial.shape[2]
    grad_zonal = np.zeros((n_edges, n_rows))
    grad_radial = np.zeros((n_edges, n_radial, channels))
    for e in range(n_edges):
        n = dst[e]
        for r in range(n_rows):
            grad_zonal[e, r] = inv[n] * math.fsum(g[n, r + 1, c] * radial[e, slots[r], c] for c in range(channels))
        for s in range(n_radial):
            rows = [r for r in range(n_rows) if slots[r] == s]
            for c in range(channels):
                grad_radial[e, s, c] = math.fsum(inv[n] * g[n, r + 1, c] * zonal[e, r] for r in rows)
    grad_inv = np.zeros(inv.shape[0])
    for n in range(inv.shape[0]):
        edges = np.nonzero(dst == n)[0]
        terms = []
        for r in range(n_rows):
            for c in range(channels):
                pre = math.fsum(zonal[e, r] * radial[e, slots[r], c] for e in edges)
                terms.append(g[n, r + 1, c] * pre)
        grad_inv[n] = math.fsum(terms)
    return grad_zonal, grad_radial, grad_inv.reshape(inv_shape)


def rmsnorm_loop(x, scale=None, eps=1e-6):
    """float64 RMSNorm row by row."""
    x = _np(x, np.float64)
    s = _np(scale, np.float64)
    rows = x.reshape(-1, x.shape[-1])
    out = np.empty_like(rows)
    for i, row in enumerate(rows):
        inv = 1.0 / math.sqrt(math.fsum(v * v for v in row) / row.shape[0] + eps)
        out[i] = row * inv * (s if s is not None else 1.0)
    return out.reshape(x.shape)


def stable_order_loop(keys):
    """Stable argsort by an explicit sort on (key, position)."""
    keys = _np(keys, np.int64)
    return np.array(sorted(range(keys.shape[0]), key=lambda i: (keys[i], i)), dtype=np.int64)


def offsets_loop(keys, n_nodes):
    keys = _np(keys, np.int64)
    offsets = [0]
    for node in range(n_nodes):
        offsets.append(offsets[-1] + int(np.count_nonzero(keys == node)))
    return np.array(offsets, dtype=np.int64)
