"""CPU oracle of the fused edge-stream elementwise chain -- test infrastructure only.

The reference has no implementation of this operator: it designs it as its
fusion candidate C4 (lipengfei1409/bysj docs/task2-hip-fusion-plan.md:280-300)
to replace eager chains of ``add_``/``mul``/``copy_`` over ``[E, R, C]``
edge tensors, with SeZM's gated activation ``act = [s * sigmoid(s),
z_r * sigmoid(q)_{g(r)}]`` (:289).  This oracle is that eager chain, in the
order the fused operator defines:

    t_k = a_k * b_k;  t_k = t_k * coef_k;  acc = t_0 + t_1 + ...  (float32, broadcasting)
    silu:  acc * sigmoid(acc)
    gate:  rows r with gate_rows[r] < 0 take silu, the others acc * sigmoid(gate[:, gate_rows[r], :])

Pinned in tests/test_oracle_pinning.py against a pure-Python loop in float64
over every element, closed values (sigmoid(0) = 1/2, silu(0) = 0), the
order of the float32 roundings, and planted mistakes.
"""
from __future__ import annotations

import torch


def edge_stream_combine_reference(terms, activation=None, gate=None, gate_rows=None) -> torch.Tensor:
    """The eager float32 chain: ``terms`` = [(coef, a) or (coef, a, b)], tensors broadcast to (E, R, C)."""
    acc = None
    for term in terms:
        coef, a = term[0], term[1]
        b = term[2] if len(term) == 3 else None
        t = a if b is None else a * b
        t = t * float(coef)
        acc = t if acc is None else acc + t
    shape = torch.broadcast_shapes(*(t.shape for term in terms for t in term[1:] if t is not None))
    acc = acc.expand(shape).contiguous()
    if activation in (None, "none"):
        return acc
    if activation == "silu":
        return acc * torch.sigmoid(acc)
    if activation != "gate":
        raise ValueError(f"unknown activation {activation!r}")
    out = torch.empty_like(acc)
    for r, g in enumerate(gate_rows):
        row = acc[:, r, :]
        if g < 0:
            out[:, r, :] = row * torch.sigmoid(row)
        else:
            q = gate.expand(shape[0], max(gate_rows) + 1, shape[2])[:, g, :]
            out[:, r, :] = row * torch.sigmoid(q)
    return out
