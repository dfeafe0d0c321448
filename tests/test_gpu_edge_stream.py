"""The fused edge-stream elementwise chain (``kernels.edge_stream``) against its oracle.

Without an activation the kernel evaluates the oracle's float32 chain in the
same order (``t = a * b; t = t * coef; acc = t_0 + t_1 + ...``), so the two
agree bit for bit, on the CPU oracle and on torch's own GPU chain; with SiLU
or SeZM's gate they agree within the float32 rule against a float64 truth.
Operands broadcast along every axis, strided and unaligned views (the scalar
path), widths that are not multiples of 4, accumulation in place, the
overlap and inference-only refusals, and empty shapes.
"""
from __future__ import annotations

import pytest
import torch

from bysj_amd.kernels import edge_stream
from oracle import edge_stream as es_ref
from parity import announce, assert_bitwise, assert_close_scaled

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _gate_rows(rows):
    """SeZM's map for R = (lmax + 1)^2 rows: row 0 scalar (silu), rows of degree l gated by gate l - 1."""
    out = []
    for r in range(rows):
        degree = int(r ** 0.5)
        out.append(-1 if degree == 0 else degree - 1)
    return out


def _case(name, seed):
    g = torch.Generator().manual_seed(seed)

    def randn(*shape):
        return torch.randn(*shape, generator=g)

    if name == "residual_gate_accumulate":  # the reference's typical chain over [E, 10, 64]
        shape = (1000, 10, 64)
        terms = [(1.0, randn(*shape)), (1.0, randn(*shape), randn(1000, 10, 1)), (1.0, randn(*shape))]
    elif name == "every_broadcast":
        shape = (333, 9, 64)
        terms = [(2.0, randn(*shape)), (-0.5, randn(64), randn(333, 1, 1)), (0.25, randn(1, 9, 64)),
                 (1.0, randn(*shape), randn(333, 1, 64))]
    elif name == "one_term":
        shape = (97, 16, 64)
        terms = [(3.0, randn(*shape))]
    elif name == "odd_channels":  # C % 4 != 0: scalar path
        shape = (257, 5, 6)
        terms = [(1.0, randn(*shape)), (0.5, randn(*shape), randn(257, 5, 1))]
    elif name == "transposed_view":  # channel stride != 1: scalar path
        shape = (200, 16, 32)
        terms = [(1.0, randn(200, 32, 16).transpose(1, 2)), (-1.0, randn(*shape))]
    elif name == "unaligned_base":  # 4-byte aligned only: scalar path
        shape = (150, 4, 64)
        flat = randn(150 * 4 * 64 + 1)
        terms = [(1.0, flat[1:].view(*shape)), (2.0, randn(*shape))]
    else:
        raise KeyError(name)
    gates = max(_gate_rows(shape[1])) + 1
    gate = randn(shape[0], max(gates, 1), shape[2])
    return shape, terms, gate


CASES = ["residual_gate_accumulate", "every_broadcast", "one_term", "odd_channels", "transposed_view",
         "unaligned_base"]


def _to_device(terms):
    return [tuple(t.to(DEV) if isinstance(t, torch.Tensor) else t for t in term) for term in terms]


@pytest.mark.parametrize("name", CASES)
@pytest.mark.parametrize("activation", [None, "silu", "gate"])
def test_edge_stream_matches_the_oracle(name, activation):
    announce("edge stream", name, activation)
    shape, terms, gate = _case(name, 3)
    rows = _gate_rows(shape[1]) if activation == "gate" else None
    q = gate if activation == "gate" else None
    got = edge_stream.edge_stream_combine(_to_device(terms), activation=activation,
                                          gate=None if q is None else q.to(DEV), gate_rows=rows)
    want = es_ref.edge_stream_combine_reference(terms, activation, q, rows)
    assert tuple(got.shape) == shape and got.is_contiguous()
    if activation is None:
        assert_bitwise(got, want, f"{name} float32 chain")
    else:
        truth = es_ref.edge_stream_combine_reference(
            [tuple(t.double() if isinstance(t, torch.Tensor) else t for t in term) for term in terms], activation,
            None if q is None else q.double(), rows)
        assert_close_scaled(got, truth, what=f"{name} {activation} vs float64")
        assert_close_scaled(got, want, what=f"{name} {activation} vs float32 chain")
    again = edge_stream.edge_stream_combine(_to_device(terms), activation=activation,
                                            gate=None if q is None else q.to(DEV), gate_rows=rows)
    assert_bitwise(again, got, f"{name} run to run")


def test_edge_stream_equals_torchs_gpu_chain():
    """Each torch op rounds once, as each step of the fused chain does: bit-identical on the same device."""
    announce("edge stream vs torch chain")
    g = torch.Generator(device=DEV).manual_seed(5)
    shape = (200_000, 10, 64)
    x, a, b = (torch.randn(*shape, generator=g, device=DEV) for _ in range(3))
    s = torch.randn(shape[0], shape[1], 1, generator=g, device=DEV)
    got = edge_stream.edge_stream_combine([(1.0, x), (0.5, a, s), (-2.0, b)])
    chain = (x * 1.0) + ((a * s) * 0.5)
    chain = chain + (b * -2.0)
    assert torch.equal(got, chain)


def test_edge_stream_accumulates_in_place_and_refuses_overlap():
    announce("edge stream in place")
    g = torch.Generator(device=DEV).manual_seed(7)
    shape = (500, 16, 64)
    acc, a = (torch.randn(*shape, generator=g, device=DEV) for _ in range(2))
    s = torch.randn(shape[0], shape[1], 1, generator=g, device=DEV)
    want = (acc * 1.0) + ((a * s) * 0.5)
    out = edge_stream.edge_stream_combine([(1.0, acc), (0.5, a, s)], out=acc)
    assert out.data_ptr() == acc.data_ptr()
    assert torch.equal(acc, want)
    # out may not overlap an operand other than as the same full-shape view
    big = torch.randn(2 * 500 * 16 * 64, device=DEV)
    shifted = big[64:64 + 500 * 16 * 64].view(*shape)
    with pytest.raises(RuntimeError, match="overlaps"):
        edge_stream.edge_stream_combine([(1.0, shifted)], out=big[:500 * 16 * 64].view(*shape))


def test_edge_stream_refusals_and_empty_shapes():
    announce("edge stream refusals")
    x = torch.randn(10, 4, 8, device=DEV)
    with pytest.raises(RuntimeError, match="inference-only"):
        edge_stream.edge_stream_combine([(1.0, x.clone().requires_grad_())])
    with torch.no_grad():
        assert edge_stream.edge_stream_combine([(1.0, x.clone().requires_grad_())]).shape == x.shape
    with pytest.raises(ValueError, match="1 to 4 terms"):
        edge_stream.edge_stream_combine([(1.0, x)] * 5)
    with pytest.raises(ValueError, match="broadcast"):
        edge_stream.edge_stream_combine([(1.0, x), (1.0, torch.randn(10, 3, 8, device=DEV))])
    with pytest.raises(ValueError, match="gate_rows"):
        edge_stream.edge_stream_combine([(1.0, x)], activation="gate", gate=x, gate_rows=[0, 0])
    with pytest.raises(TypeError, match="float32"):
        edge_stream.edge_stream_combine([(1.0, x.double())])
    empty = edge_stream.edge_stream_combine([(1.0, torch.randn(0, 4, 8, device=DEV))], activation="silu")
    assert tuple(empty.shape) == (0, 4, 8)
    # a gate activation whose rows are all silu needs no gate tensor
    silu_rows = edge_stream.edge_stream_combine([(1.0, x)], activation="gate", gate_rows=[-1] * 4)
    assert_bitwise(silu_rows, edge_stream.edge_stream_combine([(1.0, x)], activation="silu"), "all rows silu")
