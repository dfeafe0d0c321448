"""Fused edge-stream elementwise chain on gfx950.

DeepMD's SeZM blocks spend most of their elementwise time in short chains of
``add_``/``mul``/``copy_`` over ``[E, R, C]`` edge tensors (residual adds,
per-row gates, accumulations), each a separate pass over memory.  The
reference measures that pool and designs its fusion as candidate C4
(docs/task2-hip-fusion-plan.md:280-300) without implementing it: one kernel
reads the k inputs of a chain once, sums the terms of a term table (pointer,
strides, coefficient, broadcast axes) and writes one output, with an optional
activation at the end, SiLU or SeZM's gated activation
``act = [s * sigmoid(s), z_r * sigmoid(q)_{g(r)}]`` (:289).

``edge_stream_combine`` is that kernel's Python face:

    out[e, r, c] = act(sum_k (a_k[e, r, c] * b_k[e, r, c]) * coef_k)

Inference only (no autograd): an input that requires a gradient under grad
mode is refused.  Not part of ``kernels.__all__``, which stays the
reference's list, and not bound to a DeepMD seam (DeepMD's chains are not
spelled out in the reference).
"""
from __future__ import annotations

import math
import numbers

import torch

from .native import _extension, require_dcu

ACTIVATIONS = ("none", "silu", "gate")
MAX_TERMS = 4
MAX_GATE_ROWS = 64


def _term(term, k: int):
    if not isinstance(term, (tuple, list)) or len(term) not in (2, 3):
        raise TypeError(f"edge_stream_combine term {k} must be (coef, a) or (coef, a, b)")
    coef, a = term[0], term[1]
    b = term[2] if len(term) == 3 else None
    if isinstance(coef, bool) or not isinstance(coef, numbers.Real):
        raise TypeError(f"edge_stream_combine term {k}: the coefficient must be a real number")
    if not math.isfinite(float(coef)):
        raise ValueError(f"edge_stream_combine term {k}: the coefficient must be finite")
    for name, tensor in (("a", a), ("b", b)):
        if tensor is None and name == "b":
            continue
        if not isinstance(tensor, torch.Tensor):
            raise TypeError(f"edge_stream_combine term {k}: {name} must be a tensor")
        if tensor.dtype != torch.float32:
            raise TypeError(f"edge_stream_combine term {k}: {name} must be float32")
        if tensor.ndim > 3:
            raise ValueError(f"edge_stream_combine term {k}: {name} has more than three dimensions")
    return float(coef), a, b


def edge_stream_combine(terms, *, activation: str | None = None, gate=None, gate_rows=None, out=None):
    """``act(sum_k (a_k * b_k) * coef_k)`` over ``(edges, rows, channels)`` in one pass.

    ``terms``: 1 to 4 entries ``(coef, a)`` or ``(coef, a, b)``; ``a`` and
    ``b`` are float32 GPU tensors of up to three dimensions whose shapes
    broadcast (right-aligned, as in torch) to one ``(E, R, C)`` shape, the
    output's.  ``activation``: None, ``"silu"`` or ``"gate"``; the gate
    activation takes ``gate_rows`` (R ints: the gate index of each row, or
    -1 for the rows that take SiLU) and ``gate`` (broadcasting to
    ``(E, G, C)``, G = max(gate_rows) + 1).  ``out``: optional contiguous
    float32 ``(E, R, C)`` tensor; it may be a full-shape contiguous operand
    (accumulation in place) but must not overlap any other operand.

    Without an activation the result equals the eager float32 chain
    ``t = a * b; t = t * coef; acc = t_0 + t_1 + ...`` bit for bit; with one,
    it is within float32 rounding of ``acc * sigmoid(.)``.
    """
    if not isinstance(terms, (tuple, list)):
        raise TypeError("edge_stream_combine terms must be a sequence of (coef, a[, b]) tuples")
    if not 1 <= len(terms) <= MAX_TERMS:
        raise ValueError(f"edge_stream_combine takes 1 to {MAX_TERMS} terms, got {len(terms)}")
    parsed = [_term(term, k) for k, term in enumerate(terms)]
    act = "none" if activation is None else activation
    if act not in ACTIVATIONS:
        raise ValueError(f"edge_stream_combine activation must be None, 'silu' or 'gate', got {activation!r}")
    tensors = [t for _, a, b in parsed for t in (a, b) if t is not None]
    try:
        shape = torch.broadcast_shapes(*(t.shape for t in tensors))
    except RuntimeError as error:
        raise ValueError("edge_stream_combine operands do not broadcast to one shape") from error
    if len(shape) != 3:
        raise ValueError(f"edge_stream_combine operands must broadcast to (edges, rows, channels), got {tuple(shape)}")
    rows_list = None
    if act == "gate":
        if gate_rows is None or len(gate_rows) != shape[1]:
            raise ValueError("edge_stream_combine: the gate activation needs gate_rows with one entry per row")
        rows_list = [int(g) for g in gate_rows]
        if shape[1] > MAX_GATE_ROWS or any(g >= MAX_GATE_ROWS for g in rows_list):
            raise ValueError(f"edge_stream_combine: the gate activation takes at most {MAX_GATE_ROWS} rows and gates")
        if any(g >= 0 for g in rows_list):
            if not isinstance(gate, torch.Tensor) or gate.dtype != torch.float32:
                raise TypeError("edge_stream_combine: gated rows need a float32 gate tensor")
            tensors.append(gate)
    elif gate is not None or gate_rows is not None:
        raise ValueError("edge_stream_combine: gate and gate_rows belong to the gate activation")
    if out is not None:
        if not isinstance(out, torch.Tensor) or out.dtype != torch.float32:
            raise TypeError("edge_stream_combine out must be a float32 tensor")
        if tuple(out.shape) != tuple(shape) or not out.is_contiguous():
            raise ValueError(f"edge_stream_combine out must be a contiguous tensor of shape {tuple(shape)}")
        tensors.append(out)
    if torch.is_grad_enabled() and any(t.requires_grad for t in tensors):
        raise RuntimeError("edge_stream_combine is inference-only: call it under torch.no_grad() "
                           "or on tensors that do not require a gradient")
    require_dcu(*tensors)
    native = _extension("edge_stream_combine")
    return native.edge_stream_combine([(coef, a, b) for coef, a, b in parsed], tuple(shape), act,
                                      gate if act == "gate" else None, rows_list, out)


__all__ = ["edge_stream_combine", "ACTIVATIONS", "MAX_TERMS", "MAX_GATE_ROWS"]
