"""GPU parity of the GIE zonal scatter and RMSNorm (forward and backward).

Cases follow the reference's device tests (tests/csrc/accuracy/test_gie_accuracy.py,
test_rmsnorm_accuracy.py) plus the water-box configuration at a reduced size.
The GIE forward accumulates sequentially in edge order, so it is compared
with the oracle bit for bit.
"""
from __future__ import annotations

import pytest
import torch

from bysj_amd import kernels, workloads
from bysj_amd.kernels import _C
from oracle import gie as gie_ref
from oracle import loops
from oracle.rmsnorm import rmsnorm as reference_rmsnorm
from oracle.rmsnorm import rmsnorm_backward_reference
from closed_forms import gie_rmsnorm_chain_f64, rmsnorm_backward_f64, zonal_scatter_backward_f64
from parity import announce, assert_bitwise, assert_close_scaled, assert_gradient

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _fixture(degree_shape=(2,)):
    zonal = torch.tensor([[0.2, -0.1, 0.3], [0.4, 0.5, -0.2], [-0.3, 0.6, 0.1], [0.7, -0.2, 0.4]])
    radial = torch.arange(24, dtype=torch.float32).reshape(4, 2, 3) / 10
    dst = torch.tensor([1, 0, 1, 1], dtype=torch.int64)
    radial_slot = torch.tensor([0, 0, 1], dtype=torch.int64)
    inverse = torch.tensor([0.7, 0.5]).reshape(degree_shape)
    return zonal, radial, dst, radial_slot, inverse


def _to(values):
    return [value.to(DEV) for value in values]


@pytest.mark.parametrize("degree_shape", [(2,), (2, 1, 1)])
def test_gie_reference_fixture_forward_and_backward(degree_shape):
    announce("gie fixture", degree_shape)
    inputs = _fixture(degree_shape)
    zonal, radial, dst, slots, inverse = [t.to(DEV) for t in inputs]
    z = zonal.requires_grad_(True)
    r = radial.requires_grad_(True)
    inv = inverse.requires_grad_(True)
    out = kernels.zonal_scatter(z, r, dst, slots, inv)
    expected = gie_ref.zonal_scatter_reference(*inputs)
    assert_bitwise(out, expected, "forward")
    assert out[:, 0, :].count_nonzero().item() == 0
    up = torch.randn(2, 4, 3, generator=torch.Generator().manual_seed(0))
    grads = torch.autograd.grad(out, (z, r, inv), up.to(DEV))
    expected_grads = gie_ref.zonal_scatter_backward_reference(up, *inputs)
    truth = zonal_scatter_backward_f64(up, *inputs)
    for label, actual, wanted, exact in zip(("zonal", "radial", "inverse"), grads, expected_grads, truth):
        assert actual.shape == wanted.shape == exact.shape
        assert_gradient(actual, wanted, exact, f"grad {label}")


def test_gie_normalise_after_sum_known_answer_and_inverse_gradient():
    announce("gie known answer")
    zonal = torch.tensor([[1e8], [-1e8 + 8], [1.0]])
    radial = torch.ones(3, 1, 1)
    dst = torch.zeros(3, dtype=torch.int64)
    slots = torch.zeros(1, dtype=torch.int64)
    inverse = torch.tensor([0.3])
    out = kernels.zonal_scatter(*_to((zonal, radial, dst, slots, inverse)))
    expected = zonal.sum(0) * inverse
    assert_bitwise(out[0, 1], expected, "normalise after the sum")
    inv = torch.ones(1, device=DEV, requires_grad=True)
    out = kernels.zonal_scatter(zonal.to(DEV), radial.to(DEV), dst.to(DEV), slots.to(DEV), inv)
    (grad,) = torch.autograd.grad(out, (inv,), torch.tensor([[[0.0], [0.3]]], device=DEV))
    assert 2.39 <= grad.item() <= 2.71


def test_gie_empty_edges_and_range_errors():
    announce("gie empty")
    zonal = torch.empty((0, 3), device=DEV)
    radial = torch.empty((0, 2, 4), device=DEV)
    dst = torch.empty((0,), dtype=torch.int64, device=DEV)
    slots = torch.tensor([0, 0, 1], dtype=torch.int64, device=DEV)
    inverse = torch.ones((2,), device=DEV)
    out = kernels.zonal_scatter(zonal, radial, dst, slots, inverse)
    assert tuple(out.shape) == (2, 4, 4) and out.count_nonzero().item() == 0
    zonal, radial, dst, slots, inverse = _to(_fixture())
    with pytest.raises(ValueError):
        kernels.zonal_scatter(zonal, radial, torch.tensor([2, 0, 1, 1], device=DEV), slots, inverse)
    with pytest.raises(ValueError):
        kernels.zonal_scatter(zonal, radial, dst, torch.tensor([0, 2, 1], device=DEV), inverse)


@pytest.mark.parametrize("primary", [True, False])
@pytest.mark.parametrize("shuffle", [False, True])
def test_gie_water_box(primary, shuffle):
    announce("gie water", primary, shuffle)
    graph = workloads.water_graph(768, seed=2, rcut=3.0)
    case = workloads.gie_config(graph, seed=2, primary=primary, channels=64)
    dst = case["dst"]
    zonal, radial = case["zonal"], case["radial"]
    if shuffle:
        perm = torch.randperm(dst.numel(), generator=torch.Generator().manual_seed(4))
        dst, zonal, radial = dst[perm].contiguous(), zonal[perm].contiguous(), radial[perm].contiguous()
    inputs = (zonal, radial, dst, case["radial_slot"], case["inv_sqrt_deg"])
    z, r = zonal.to(DEV).requires_grad_(True), radial.to(DEV).requires_grad_(True)
    inv = case["inv_sqrt_deg"].to(DEV).requires_grad_(True)
    out = kernels.zonal_scatter(z, r, dst.to(DEV), case["radial_slot"].to(DEV), inv)
    assert_bitwise(out, gie_ref.zonal_scatter_reference(*inputs), "forward")
    up = torch.randn(out.shape, generator=torch.Generator().manual_seed(1))
    grads = torch.autograd.grad(out, (z, r, inv), up.to(DEV))
    expected = gie_ref.zonal_scatter_backward_reference(up, *inputs)
    truth = zonal_scatter_backward_f64(up, *inputs)
    for label, actual, wanted, exact in zip(("zonal", "radial", "inverse"), grads, expected, truth):
        assert_gradient(actual, wanted, exact, f"grad {label}")


def test_gie_forward_against_fp64_truth():
    announce("gie fp64 truth")
    graph = workloads.water_graph(600, seed=5, rcut=3.0)
    case = workloads.gie_config(graph, seed=5, primary=False, channels=8)
    inputs = (case["zonal"], case["radial"], case["dst"], case["radial_slot"], case["inv_sqrt_deg"])
    out = kernels.zonal_scatter(*_to(inputs))
    assert_close_scaled(out, loops.zonal_scatter_loop(*inputs), what="vs fp64 truth")


def test_gie_current_stream():
    announce("gie stream")
    stream = torch.cuda.Stream()
    inputs = _fixture()
    with torch.cuda.stream(stream):
        out = kernels.zonal_scatter(*_to(inputs))
    torch.cuda.current_stream().wait_stream(stream)
    assert_bitwise(out, gie_ref.zonal_scatter_reference(*inputs), "side stream")


# ---------------------------------------------------------------------------
# RMSNorm
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("shape", [(1, 1), (7, 127), (2, 3, 257), (0, 65), (5, 1024), (3, 4096), (2, 5000)])
def test_rmsnorm_forward_tail_widths(shape):
    announce("rmsnorm fwd", shape)
    gen = torch.Generator().manual_seed(len(shape) + shape[-1])
    x = torch.randn(*shape, generator=gen)
    scale = torch.randn(shape[-1], generator=gen)
    out = kernels.rmsnorm(x.to(DEV), scale.to(DEV), eps=1e-5)
    assert tuple(out.shape) == shape
    assert_close_scaled(out, reference_rmsnorm(x, scale, eps=1e-5), what="vs oracle")
    if x.numel():
        assert_close_scaled(out, loops.rmsnorm_loop(x, scale, 1e-5), what="vs fp64 truth")


@pytest.mark.parametrize("shape", [(5, 3, 127), (64, 1024), (9, 5000)])
def test_rmsnorm_gradients(shape):
    announce("rmsnorm bwd", shape)
    gen = torch.Generator().manual_seed(shape[-1])
    x = torch.randn(*shape, generator=gen)
    scale = torch.randn(shape[-1], generator=gen)
    up = torch.randn(*shape, generator=gen)
    xd = x.to(DEV).requires_grad_(True)
    sd = scale.to(DEV).requires_grad_(True)
    out = kernels.rmsnorm(xd, sd, eps=1e-5)
    grads = torch.autograd.grad(out, (xd, sd), up.to(DEV))
    e_x, e_s = rmsnorm_backward_reference(up, x, scale, eps=1e-5)
    t_x, t_s = rmsnorm_backward_f64(up, x, scale, eps=1e-5)
    assert_gradient(grads[0], e_x, t_x, "grad_x")
    assert_gradient(grads[1], e_s, t_s, "grad_scale")
    again = torch.autograd.grad(kernels.rmsnorm(xd, sd, eps=1e-5), (xd, sd), up.to(DEV))
    assert_bitwise(again[1], grads[1], "grad_scale run-to-run")


def test_rmsnorm_zero_input_no_scale_and_stream():
    announce("rmsnorm zero/stream")
    x = torch.zeros(2, 7, device=DEV)
    out = kernels.rmsnorm(x, eps=1e-6)
    assert torch.equal(out, x)
    stream = torch.cuda.Stream()
    gen = torch.Generator().manual_seed(3)
    xs, ss = torch.randn(9, 131, generator=gen), torch.randn(131, generator=gen)
    with torch.cuda.stream(stream):
        out = kernels.rmsnorm(xs.to(DEV), ss.to(DEV))
    torch.cuda.current_stream().wait_stream(stream)
    assert_close_scaled(out, reference_rmsnorm(xs, ss), what="side stream")
    # a scale gradient needs a scale (csrc/rmsnorm.cpp:138-139 of the reference)
    empty = torch.empty(0, device=DEV)
    y, inverse_rms = _C.rmsnorm_forward(xs.to(DEV), empty, 1e-6)
    with pytest.raises(RuntimeError, match="scale is omitted"):
        _C.rmsnorm_backward(torch.ones_like(y), xs.to(DEV), empty, inverse_rms, True)
    grad_x, grad_scale = _C.rmsnorm_backward(torch.ones_like(y), xs.to(DEV), empty, inverse_rms, False)
    assert grad_scale.numel() == 0
    e_x, _ = rmsnorm_backward_reference(torch.ones(9, 131), xs, None, 1e-6)
    t_x, _ = rmsnorm_backward_f64(torch.ones(9, 131), xs, None, 1e-6)
    assert_gradient(grad_x, e_x, t_x, "grad_x without scale")


def test_gie_then_rmsnorm_config3_reduced():
    announce("gie+rmsnorm config3 reduced")
    graph = workloads.water_graph(1200, seed=0)
    case = workloads.gie_config(graph, seed=0, primary=True, channels=64)
    inputs = (case["zonal"], case["radial"], case["dst"], case["radial_slot"], case["inv_sqrt_deg"])
    out = kernels.zonal_scatter(*_to(inputs))
    expected = gie_ref.zonal_scatter_reference(*inputs)
    assert_bitwise(out, expected, "gie")
    rows = out.reshape(out.shape[0], -1)
    y = kernels.rmsnorm(rows, case["rms_scale"].to(DEV), eps=1e-6)
    assert_close_scaled(y, reference_rmsnorm(expected.reshape(expected.shape[0], -1), case["rms_scale"], 1e-6),
                        what="rmsnorm")


# ---------------------------------------------------------------------------
# fused GIE -> RMSNorm (extension: kernels.gie.gie_zonal_scatter_rmsnorm)
# ---------------------------------------------------------------------------

def _oracle_gie_rmsnorm(zonal, radial, dst, slots, inverse, scale, eps):
    rows = gie_ref.zonal_scatter_reference(zonal, radial, dst, slots, inverse)
    flat = rows.reshape(rows.shape[0], -1)
    return reference_rmsnorm(flat, scale, eps).reshape(rows.shape)


@pytest.mark.parametrize("primary", [True, False])
@pytest.mark.parametrize("use_scale", [True, False])
@pytest.mark.parametrize("shuffle", [False, True])
def test_gie_rmsnorm_fused_matches_two_operators(primary, use_scale, shuffle):
    """Fused forward == zonal_scatter then rmsnorm (both gfx950) bit for bit; both within the fp32
    rule of the oracle chain; gradients of every input against autograd through the oracle."""
    from bysj_amd.kernels import gie as gie_ops

    announce("gie rmsnorm fused", primary, use_scale, shuffle)
    graph = workloads.water_graph(768, seed=5, rcut=3.0)
    case = workloads.gie_config(graph, seed=5, primary=primary, channels=64)
    dst, zonal, radial = case["dst"], case["zonal"], case["radial"]
    if shuffle:
        perm = torch.randperm(dst.numel(), generator=torch.Generator().manual_seed(6))
        dst, zonal, radial = dst[perm].contiguous(), zonal[perm].contiguous(), radial[perm].contiguous()
    scale = case["rms_scale"] if use_scale else None
    inputs = (zonal, radial, dst, case["radial_slot"], case["inv_sqrt_deg"])
    d = _to(inputs)
    ds = None if scale is None else scale.to(DEV)
    with torch.no_grad():
        fused = gie_ops.gie_zonal_scatter_rmsnorm(*d, scale=ds, eps=1e-6)
        rows = kernels.zonal_scatter(*d)
        two_step = kernels.rmsnorm(rows.reshape(rows.shape[0], -1), ds, eps=1e-6).reshape(rows.shape)
    assert_bitwise(fused, two_step, "fused vs zonal_scatter -> rmsnorm")
    assert_close_scaled(fused, _oracle_gie_rmsnorm(*inputs, scale, 1e-6), what="fused vs oracle")
    again = gie_ops.gie_zonal_scatter_rmsnorm(*d, scale=ds, eps=1e-6)
    assert_bitwise(again, fused, "run to run")

    z, r = d[0].clone().requires_grad_(True), d[1].clone().requires_grad_(True)
    inv = d[4].clone().requires_grad_(True)
    s = None if ds is None else ds.clone().requires_grad_(True)
    out = gie_ops.gie_zonal_scatter_rmsnorm(z, r, d[2], d[3], inv, scale=s, eps=1e-6)
    assert_bitwise(out, fused, "forward with gradients kept")
    up = torch.randn(out.shape, generator=torch.Generator().manual_seed(7))
    wrt = (z, r, inv) + (() if s is None else (s,))
    grads = torch.autograd.grad(out, wrt, up.to(DEV))
    cz, cr = inputs[0].clone().requires_grad_(True), inputs[1].clone().requires_grad_(True)
    cinv = inputs[4].clone().requires_grad_(True)
    cs = None if scale is None else scale.clone().requires_grad_(True)
    expected_out = _oracle_gie_rmsnorm(cz, cr, inputs[2], inputs[3], cinv, cs, 1e-6)
    expected = torch.autograd.grad(expected_out, (cz, cr, cinv) + (() if cs is None else (cs,)), up)
    truth, terms = gie_rmsnorm_chain_f64(inputs, scale, up, 1e-6)
    for label, actual, wanted, exact in zip(("zonal", "radial", "inverse", "scale"), grads, expected, truth):
        if label == "inverse":
            continue
        assert_gradient(actual, wanted, exact, f"grad {label}")
    # RMSNorm is scale invariant, so d y / d inv_sqrt_deg is a sum of (n_rows + 1) * channels terms
    # that cancel (exactly, but for eps): fp32 results are rounding noise around a tiny value, and
    # max|ref| says nothing about their size.  Check it against the chain in float64, to 1e-5 of
    # the node's sum of absolute terms (the fp32 rule's relative bar, on the terms that are summed).
    error = (grads[2].double().cpu() - truth[2]).abs()
    assert bool((error <= 1e-5 * terms + 1e-12).all()), f"grad inverse: worst {float((error / terms).max())}"


def test_gie_rmsnorm_unfused_shapes_and_empty_edges():
    """Rows the fused kernel does not take (channels % 4 != 0) and graphs without edges run the two
    operators; results still follow the oracle chain."""
    from bysj_amd.kernels import gie as gie_ops

    announce("gie rmsnorm unfused shapes")
    inputs = _fixture()
    width = (inputs[0].shape[1] + 1) * inputs[1].shape[2]
    scale = torch.linspace(0.5, 1.5, width)
    out = gie_ops.gie_zonal_scatter_rmsnorm(*_to(inputs), scale=scale.to(DEV), eps=1e-6)
    assert_close_scaled(out, _oracle_gie_rmsnorm(*inputs, scale, 1e-6), what="3 channels")
    zonal = torch.empty(0, 15)
    radial = torch.empty(0, 16, 8)
    dst = torch.empty(0, dtype=torch.int64)
    slots = torch.arange(1, 16, dtype=torch.int64)
    inverse = torch.ones(3)
    out = gie_ops.gie_zonal_scatter_rmsnorm(*_to((zonal, radial, dst, slots, inverse)), eps=1e-6)
    assert out.shape == (3, 16, 8) and out.count_nonzero().item() == 0
    with pytest.raises(ValueError):
        gie_ops.gie_zonal_scatter_rmsnorm(*_to(inputs), scale=torch.ones(3, device=DEV), eps=1e-6)
    with pytest.raises(ValueError):
        gie_ops.gie_zonal_scatter_rmsnorm(*_to(inputs), eps=0.0)


# ---------------------------------------------------------------------------
# shared radial slots: the per-slot kernels against the oracle and the kernels
# that assume nothing about the slot map (slot_info = 0)
# ---------------------------------------------------------------------------

_DEEPMD_SLOTS = [0, 0, 0, 1, 1, 1, 1, 1, 2, 2, 2, 2, 2, 2, 2]
_SHARED_LAYOUTS = [
    # (radial_slot, n_radial, channels): what each exercises
    (_DEEPMD_SLOTS, 3, 64),        # DeepMD rows l = 1..3: 7 rows on one slot; backward 8 lanes per slot
    ([0, 0, 1, 1], 2, 16),         # at most 4 rows per slot; backward 2 lanes per slot
    ([1, 0, 1, 0, 1], 3, 32),      # slot 2 unreferenced: its gradient is written as zeros
    ([0] * 8 + [1], 2, 128),       # 8 rows on one slot; backward 16 lanes per slot, 2 edges per wave step
    ([0] * 9, 1, 64),              # 9 rows on one slot: beyond the per-slot kernels, general kernels
    (_DEEPMD_SLOTS, 3, 128),       # forward pairs past one per lane (96)
    (_DEEPMD_SLOTS, 3, 256),       # forward beyond the shared layout; backward general (32 lanes per slot)
    (_DEEPMD_SLOTS, 3, 8),         # one lane per slot, 21 edges per wave step (backward)
    (_DEEPMD_SLOTS, 3, 20),        # channels % 8 != 0: forward shared, backward general
    (_DEEPMD_SLOTS, 3, 6),         # channels % 4 != 0: scalar kernels
    ([0] * 3 + [1] * 5 + [2] * 7 + [3] * 9, 4, 64),  # lmax = 4: 24 rows, 9 on one slot; backward edge lanes
    ([2, 0, 1, 2, 0, 1, 1, 2, 0, 2], 3, 64),         # rows of a slot interleaved with the others' (backward order)
    ([1, 1, 0, 1, 1, 0, 1], 2, 128),                 # 16 lanes per edge, 4 edges per wave step
]


def _shared_slot_case(slots, n_radial, channels, shuffle, seed=41):
    generator = torch.Generator().manual_seed(seed)
    n_nodes = 48
    degrees = torch.poisson(torch.full((n_nodes,), 6.0), generator=generator).to(torch.int64)
    degrees[3] = 0
    degrees[10] = 301  # several wave steps and an uneven tail
    dst = torch.repeat_interleave(torch.arange(n_nodes), degrees)
    edges, rows = dst.numel(), len(slots)
    zonal = torch.randn((edges, rows), generator=generator)
    radial = torch.randn((edges, n_radial, channels), generator=generator)
    inverse = torch.rsqrt(degrees.to(torch.float32) + 1.0)
    if shuffle:
        perm = torch.randperm(edges, generator=generator)
        dst, zonal, radial = dst[perm].contiguous(), zonal[perm].contiguous(), radial[perm].contiguous()
    return zonal, radial, dst, torch.tensor(slots, dtype=torch.int64), inverse


@pytest.mark.parametrize("shuffle", [False, True], ids=["sorted", "shuffled"])
@pytest.mark.parametrize("layout", _SHARED_LAYOUTS, ids=lambda v: f"{max(v[0].count(s) for s in set(v[0]))}rows-S{v[1]}-C{v[2]}")
def test_gie_shared_slot_layouts(layout, shuffle):
    slots, n_radial, channels = layout
    announce("gie shared slots", slots, n_radial, channels, shuffle)
    inputs = _shared_slot_case(slots, n_radial, channels, shuffle)
    zonal, radial, dst, radial_slot, inverse = _to(inputs)
    offsets, order, info = _C.gie_group(dst, radial_slot, inverse.numel(), n_radial)
    most = max(slots.count(s) for s in set(slots))
    assert (info >> 16) & 0xFF == most and not info & 2

    # forward: both kernel families equal the sequential oracle bit for bit
    expected = gie_ref.zonal_scatter_reference(*inputs)
    out = _C.gie_zonal_scatter_forward_csr(zonal, radial, offsets, order, radial_slot, inverse, info)
    assert_bitwise(out, expected, "forward, slot-aware kernel")
    plain = _C.gie_zonal_scatter_forward_csr(zonal, radial, offsets, order, radial_slot, inverse, 0)
    assert_bitwise(plain, expected, "forward, slot-agnostic kernel")

    # backward through the operator, against the oracle's autograd and the fp64 closed form
    up = torch.randn(expected.shape, generator=torch.Generator().manual_seed(5))
    z, r = zonal.clone().requires_grad_(True), radial.clone().requires_grad_(True)
    inv = inverse.clone().requires_grad_(True)
    out = kernels.zonal_scatter(z, r, dst, radial_slot, inv)
    assert_bitwise(out, expected, "operator forward")
    grads = torch.autograd.grad(out, (z, r, inv), up.to(DEV))
    oracle = gie_ref.zonal_scatter_backward_reference(up, *inputs)
    truth = zonal_scatter_backward_f64(up, *inputs)
    for label, actual, wanted, exact in zip(("zonal", "radial", "inverse"), grads, oracle, truth):
        assert_gradient(actual, wanted, exact, f"grad {label}, slot-aware kernel")
    plain = _C.gie_zonal_scatter_backward_csr(up.to(DEV), zonal, radial, offsets, order, radial_slot, inverse, 0)
    for label, actual, wanted, exact in zip(("zonal", "radial", "inverse"), plain, oracle, truth):
        assert_gradient(actual, wanted, exact, f"grad {label}, slot-agnostic kernel")
    again = _C.gie_zonal_scatter_backward_csr(up.to(DEV), zonal, radial, offsets, order, radial_slot, inverse, info)
    for label, first, second in zip(("zonal", "radial", "inverse"), grads, again):
        assert_bitwise(second, first, f"grad {label} run to run")


def test_gie_shared_slot_kernels_skip_absent_outputs():
    announce("gie shared slots, partial outputs")
    inputs = _shared_slot_case(_DEEPMD_SLOTS, 3, 64, shuffle=True)
    zonal, radial, dst, radial_slot, inverse = _to(inputs)
    offsets, order, info = _C.gie_group(dst, radial_slot, inverse.numel(), 3)
    up = torch.randn((inverse.numel(), 16, 64), generator=torch.Generator().manual_seed(6)).to(DEV)
    full = _C.gie_zonal_scatter_backward_csr(up, zonal, radial, offsets, order, radial_slot, inverse, info)
    for need in ((True, False, False), (False, True, False), (False, False, True)):
        part = _C.gie_zonal_scatter_backward_csr(up, zonal, radial, offsets, order, radial_slot, inverse, info,
                                                 need=need)
        for wanted, got, reference in zip(need, part, full):
            if wanted:
                assert_bitwise(got, reference, f"partial outputs {need}")
            else:
                assert got is None
