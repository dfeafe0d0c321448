"""Pins the CPU oracle (oracle/) before any GPU result is compared with it.

Three kinds of checks, all on the CPU:

1. the reference's own known-answer cases (tests/golden/known_answers.json,
   expectations from exact-sum loops and closed forms, not from the oracle);
2. brute force on small random inputs (``oracle.loops``: float64 with
   ``math.fsum``, or the float32 edge-ordered loop for bit-exact sums) and
   the invariants the mathematics fixes (sum-to-one, masking, Newton's third
   law, stable grouping);
3. planted mistakes: each check is run once more on a deliberately broken
   copy of the oracle function (a dropped term, a wrong sign, a transposed
   operand, normalising before the sum, an unstable sort) and must reject it,
   which shows the checks above can fail.
"""
from __future__ import annotations

import importlib
import math

import numpy as np
import pytest
import torch

import closed_forms
from golden_cases import load_cases
from oracle import edge_stream as es_ref
from oracle import gie as gie_ref
from oracle import loops
from oracle import segment as ref
from parity import assert_bitwise, assert_close_scaled

rms_ref = importlib.import_module("oracle.rmsnorm")  # the package re-exports a function of the same name


# ---------------------------------------------------------------------------
# reusable checks (taking the implementation under test)
# ---------------------------------------------------------------------------

def check_offsets(segment_offsets, group_by_source):
    for case in load_cases("segment_offsets"):
        got = segment_offsets(case["dst"], case["n_nodes"])
        assert_bitwise(got, case["offsets"], case["name"])
        assert_bitwise(got, case["closed_form"], case["name"] + " closed form")
    for case in load_cases("group_by_source"):
        order, offsets = group_by_source(case["src"], case["n_nodes"])
        assert_bitwise(order, case["order"], case["name"] + " order")
        assert_bitwise(order, case["closed_form_order"], case["name"] + " closed form order")
        assert_bitwise(offsets, case["offsets"], case["name"] + " offsets")
        assert_bitwise(offsets, case["closed_form_offsets"], case["name"] + " closed form offsets")


def check_segment_sum(segment_sum):
    for case in load_cases("segment_sum"):
        out = segment_sum(case["src"], case["dst"], case["offsets"], case["edge_scale"], case["node_scale"])
        assert_bitwise(out, case["out_f32_sequential"], case["name"] + " sequential float32")
        assert_close_scaled(out, case["out_f64"], what=case["name"] + " vs exact sum")
        if isinstance(case.get("closed_form"), torch.Tensor):
            assert_bitwise(out, case["closed_form"], case["name"] + " closed form")


def check_segment_sum_backward(backward):
    for case in load_cases("segment_sum_backward"):
        grad_src, grad_edge, grad_node = backward(case["grad_out"], case["src"], case["dst"], case["offsets"],
                                                  case["edge_scale"], case["node_scale"])
        assert_close_scaled(grad_src, case["grad_src_f64"], what="grad_src")
        assert_close_scaled(grad_edge, case["grad_edge_scale_f64"], what="grad_edge_scale")
        assert_close_scaled(grad_node, case["grad_node_scale_f64"], what="grad_node_scale")


def check_segment_softmax(softmax):
    for case in load_cases("segment_softmax"):
        alpha, null_alpha = softmax(case["logit"], case["env"], case["dst"], case["offsets"], case["null_logit"])
        assert_close_scaled(alpha, case["alpha_f64"], what=case["name"] + " alpha")
        if case["null_logit"] is None:
            assert null_alpha is None
        else:
            assert_close_scaled(null_alpha, case["null_alpha_f64"], what=case["name"] + " null_alpha")


def check_segment_softmax_backward(backward):
    for case in load_cases("segment_softmax_backward"):
        grad_logit, grad_env, grad_null = backward(case["grad_alpha"], case["logit"], case["env"], case["dst"],
                                                   case["offsets"], case["null_logit"], case["grad_null_alpha"])
        assert_close_scaled(grad_logit, case["grad_logit_f64"], what="grad_logit")
        assert_close_scaled(grad_null, case["grad_null_logit_f64"], what="grad_null_logit")
        assert_close_scaled(grad_env, case["grad_env_f64"], what="grad_env")


def check_force(force_assembly):
    for case in load_cases("force_assembly"):
        force, virial = force_assembly(case["grad_edge"], case["edge_vec"], case["src"], case["dst"],
                                       case["dst_offsets"], case["src_offsets"])
        assert_close_scaled(force, case["force_f64"], what=case["name"] + " force")
        assert_close_scaled(virial, case["virial_f64"], what=case["name"] + " virial")
        assert float(force.double().sum(0).abs().max()) <= 1e-6


def check_gie(zonal_scatter):
    for case in load_cases("zonal_scatter"):
        out = zonal_scatter(case["zonal"], case["radial"], case["dst"], case["radial_slot"], case["inv_sqrt_deg"])
        assert_close_scaled(out, case["out_f64"], what=case["name"])
        assert int(out[:, 0, :].count_nonzero()) == 0
        if "exact_f32_row1" in case:
            assert_bitwise(out[0, 1], case["exact_f32_row1"], "normalise after the destination sum")


def check_gie_backward(backward):
    for case in load_cases("zonal_scatter_backward"):
        grad_zonal, grad_radial, grad_inv = backward(case["grad_output"], case["zonal"], case["radial"], case["dst"],
                                                     case["radial_slot"], case["inv_sqrt_deg"])
        assert_close_scaled(grad_zonal, case["grad_zonal_f64"], what=case["name"] + " grad_zonal")
        assert_close_scaled(grad_radial, case["grad_radial_f64"], what=case["name"] + " grad_radial")
        assert tuple(grad_inv.shape) == tuple(case["inv_sqrt_deg"].shape), case["name"] + " grad_inv shape"
        assert_close_scaled(grad_inv, case["grad_inv_sqrt_deg_f64"], what=case["name"] + " grad_inv_sqrt_deg")


def check_rmsnorm(rmsnorm):
    for case in load_cases("rmsnorm"):
        out = rmsnorm(case["x"], case["scale"], case["eps"])
        assert_close_scaled(out, case["out_f64"], what=case["name"])
        assert bool(torch.isfinite(out).all())


def _edge_stream_case(seed):
    """Operands of every broadcast shape the fused chain takes, over (E, R, C) = (3, 4, 5)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(3, 4, 5, generator=g)
    a = torch.randn(3, 4, 5, generator=g)
    s = torch.randn(3, 4, 1, generator=g)      # per (edge, row), broadcast over channels
    w = torch.randn(5, generator=g)            # per channel, broadcast over edges and rows
    e = torch.randn(3, 1, 1, generator=g)      # per edge
    terms = [(1.0, x), (-0.75, a, s), (1.5, w, e), (0.3, a)]
    q = torch.randn(3, 2, 5, generator=g)      # two gates per edge and channel
    gate_rows = [-1, 0, 1, 1]
    return terms, q, gate_rows


def _edge_stream_loops(terms, activation, gate, gate_rows, shape, exact_f32):
    """Element by element: float32 scalar arithmetic in the chain's order (exact_f32), else float64."""
    cast = np.float32 if exact_f32 else float
    out = np.zeros(shape, dtype=np.float32 if exact_f32 else np.float64)
    views = []
    for term in terms:
        b = term[2] if len(term) == 3 else None
        views.append((cast(term[0]), term[1].expand(shape).numpy(), None if b is None else b.expand(shape).numpy()))
    for e, r, c in np.ndindex(*shape):
        acc = None
        for coef, a, b in views:
            t = cast(a[e, r, c]) if b is None else cast(a[e, r, c]) * cast(b[e, r, c])
            t = t * coef
            acc = t if acc is None else acc + t
        if activation == "silu" or (activation == "gate" and gate_rows[r] < 0):
            acc = acc / (1.0 + math.exp(-float(acc)))
        elif activation == "gate":
            acc = acc / (1.0 + math.exp(-float(gate[e, gate_rows[r], c])))
        out[e, r, c] = acc
    return torch.from_numpy(out)


def check_edge_stream(combine):
    for seed in (0, 1):
        terms, q, gate_rows = _edge_stream_case(seed)
        shape = (3, 4, 5)
        plain = combine(terms)
        assert_bitwise(plain, _edge_stream_loops(terms, None, None, None, shape, True), "edge stream float32 order")
        for activation in ("silu", "gate"):
            got = combine(terms, activation, q, gate_rows)
            want = _edge_stream_loops(terms, activation, q, gate_rows, shape, False)
            assert_close_scaled(got, want, what=f"edge stream {activation}")
        # closed values: sigmoid(0) = 1/2 on the gated rows, silu(0) = 0
        zero_gate = combine(terms, "gate", torch.zeros_like(q), gate_rows)
        assert_bitwise(zero_gate[:, 1:], plain[:, 1:] * 0.5, "edge stream gate at sigmoid(0)")
        zeros = combine([(1.0, torch.zeros(3, 4, 5))], "silu")
        assert int(zeros.count_nonzero()) == 0


# ---------------------------------------------------------------------------
# 1. the oracle against the known answers
# ---------------------------------------------------------------------------

def test_csr_helpers_known_answers():
    check_offsets(ref.segment_offsets, ref.group_by_source)


def test_segment_sum_known_answers():
    check_segment_sum(ref.segment_sum_reference)


def test_segment_sum_backward_closed_form():
    check_segment_sum_backward(ref.segment_sum_backward_reference)


def test_segment_softmax_known_answers():
    check_segment_softmax(ref.segment_softmax_reference)


def test_segment_softmax_backward_closed_form():
    check_segment_softmax_backward(ref.segment_softmax_backward_reference)


def test_force_assembly_known_answers():
    check_force(ref.force_assembly_reference)


def test_gie_known_answers():
    check_gie(gie_ref.zonal_scatter_reference)


def test_gie_backward_closed_form():
    check_gie_backward(gie_ref.zonal_scatter_backward_reference)


def test_rmsnorm_known_answers():
    check_rmsnorm(rms_ref.rmsnorm)


# ---------------------------------------------------------------------------
# 2. brute force and invariants on small random inputs
# ---------------------------------------------------------------------------

def _random_graph(seed, nodes=9, max_degree=7, empty_every=4):
    gen = np.random.default_rng(seed)
    degrees = gen.integers(0, max_degree + 1, size=nodes)
    degrees[::empty_every] = 0
    dst = np.repeat(np.arange(nodes), degrees)
    return torch.from_numpy(dst.astype(np.int64)), ref.segment_offsets(torch.from_numpy(dst.astype(np.int64)), nodes)


@pytest.mark.parametrize("seed", range(4))
def test_csr_helpers_brute_force(seed):
    gen = torch.Generator().manual_seed(seed)
    keys = torch.randint(0, 11, (200,), generator=gen)
    assert_bitwise(ref.segment_offsets(keys, 11), torch.from_numpy(loops.offsets_loop(keys, 11)), "offsets")
    order, offsets = ref.group_by_source(keys, 11)
    assert_bitwise(order, torch.from_numpy(loops.stable_order_loop(keys)), "stable order")
    assert_bitwise(offsets, torch.from_numpy(loops.offsets_loop(keys, 11)), "offsets")
    with pytest.raises(ValueError):
        ref.segment_offsets(torch.tensor([0, 11]), 11)
    with pytest.raises(ValueError):
        ref.group_by_source(torch.tensor([-1]), 11)


@pytest.mark.parametrize("seed", range(3))
@pytest.mark.parametrize("channels", [1, 5, 16])
def test_segment_sum_brute_force(seed, channels):
    dst, offsets = _random_graph(seed)
    gen = torch.Generator().manual_seed(seed)
    src = torch.randn(dst.numel(), channels, generator=gen)
    w = torch.rand(dst.numel(), generator=gen) + 0.5
    s = torch.rand(offsets.numel() - 1, generator=gen) + 0.5
    out = ref.segment_sum_reference(src, dst, offsets, w, s)
    sequential = loops.segment_sum_sequential_f32(src, dst, offsets.numel() - 1, w, s)
    assert_bitwise(out, torch.from_numpy(sequential), "sequential float32 loop")
    assert_close_scaled(out, loops.segment_sum_loop(src, dst, offsets.numel() - 1, w, s), what="exact sum")
    with pytest.raises(ValueError):
        bad = offsets.clone()
        bad[1] += 1
        ref.segment_sum_reference(src, dst, bad)


def _softmax_inputs(seed, channels=4, masked_fraction=0.2, big=True):
    dst, offsets = _random_graph(seed, nodes=8, max_degree=9)
    gen = torch.Generator().manual_seed(100 + seed)
    edges = dst.numel()
    logit = torch.randn(edges, channels, generator=gen) * 2.0
    if big and edges:
        logit[0, 0] = 40.0
        logit[-1, -1] = -40.0
    env = torch.rand(edges, generator=gen) + 0.1
    env[torch.rand(edges, generator=gen) < masked_fraction] = -0.5
    null = torch.randn(offsets.numel() - 1, channels, generator=gen)
    return logit, env, dst, offsets, null


@pytest.mark.parametrize("seed", range(4))
@pytest.mark.parametrize("with_null", [False, True])
def test_segment_softmax_brute_force_and_invariants(seed, with_null):
    logit, env, dst, offsets, null = _softmax_inputs(seed)
    null = null if with_null else None
    n_nodes = offsets.numel() - 1
    alpha, null_alpha = ref.segment_softmax_reference(logit, env, dst, offsets, null)
    e_alpha, e_null = loops.segment_softmax_loop(logit, env, dst, n_nodes, null)
    assert_close_scaled(alpha, e_alpha, what="alpha vs per-segment loop")
    assert int(alpha[env <= 0].count_nonzero()) == 0, "masked edges carry mass"
    totals = torch.zeros(n_nodes, logit.shape[1]).index_add_(0, dst, alpha)
    if with_null:
        assert_close_scaled(null_alpha, e_null, what="null_alpha vs loop")
        totals = totals + null_alpha
        torch.testing.assert_close(totals, torch.ones_like(totals), rtol=1e-5, atol=1e-6)
    else:
        live = torch.zeros(n_nodes).index_add_(0, dst, (env > 0).float()) > 0
        torch.testing.assert_close(totals[live], torch.ones_like(totals[live]), rtol=1e-5, atol=1e-6)
        assert int(totals[~live].count_nonzero()) == 0, "a segment without mass must give zeros"


def test_segment_softmax_special_cases():
    dst = torch.tensor([0, 0, 1], dtype=torch.int64)
    offsets = torch.tensor([0, 2, 3, 3], dtype=torch.int64)
    logit = torch.randn(3, 2, generator=torch.Generator().manual_seed(0))
    env = torch.tensor([-1.0, 0.0, float("nan")])
    null = torch.randn(3, 2, generator=torch.Generator().manual_seed(1))
    alpha, null_alpha = ref.segment_softmax_reference(logit, env, dst, offsets, null)
    assert int(alpha.count_nonzero()) == 0
    torch.testing.assert_close(null_alpha, torch.ones(3, 2))  # null alone takes all the mass
    alpha, none = ref.segment_softmax_reference(logit, env, dst, offsets)
    assert none is None and int(alpha.count_nonzero()) == 0  # no mass anywhere -> zeros


@pytest.mark.parametrize("seed", range(3))
def test_segment_sum_and_softmax_backward_closed_forms_random(seed):
    dst, offsets = _random_graph(seed)
    n_nodes, edges = offsets.numel() - 1, dst.numel()
    gen = torch.Generator().manual_seed(seed + 50)
    src = torch.randn(edges, 3, generator=gen)
    w = torch.rand(edges, generator=gen) + 0.5
    s = torch.rand(n_nodes, generator=gen) + 0.5
    g = torch.randn(n_nodes, 3, generator=gen)
    grad_src, grad_w, grad_s = ref.segment_sum_backward_reference(g, src, dst, offsets, w, s)
    gd, sd, wd, nd = g.double(), src.double(), w.double(), s.double()
    expected_src = gd[dst] * nd[dst, None] * wd[:, None]
    expected_w = (gd[dst] * nd[dst, None] * sd).sum(1)
    prefix = torch.from_numpy(loops.segment_sum_loop(src, dst, n_nodes, w))
    expected_s = (gd * prefix).sum(1)
    assert_close_scaled(grad_src, expected_src, what="grad_src")
    assert_close_scaled(grad_w, expected_w, what="grad_edge_scale")
    assert_close_scaled(grad_s, expected_s, what="grad_node_scale")

    logit, env, dst, offsets, null = _softmax_inputs(seed, big=False, masked_fraction=0.0)
    alpha, null_alpha = ref.segment_softmax_reference(logit, env, dst, offsets, null)
    ga = torch.randn(alpha.shape, generator=gen)
    gn = torch.randn(null_alpha.shape, generator=gen)
    grad_logit, grad_env, grad_null = ref.segment_softmax_backward_reference(ga, logit, env, dst, offsets, null, gn)
    a64, n64 = loops.segment_softmax_loop(logit, env, dst, offsets.numel() - 1, null)
    a64, n64 = torch.from_numpy(a64), torch.from_numpy(n64)
    expectation = torch.zeros_like(n64).index_add_(0, dst, a64 * ga.double()) + n64 * gn.double()
    expected_logit = a64 * (ga.double() - expectation[dst])
    assert_close_scaled(grad_logit, expected_logit, what="grad_logit")
    assert_close_scaled(grad_null, n64 * (gn.double() - expectation), what="grad_null")
    assert_close_scaled(grad_env, expected_logit.sum(1) * 2.0 / env.double(), what="grad_env")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_force_assembly_brute_force(dtype):
    dst, dst_offsets = _random_graph(7, nodes=10)
    gen = torch.Generator().manual_seed(7)
    src = torch.randint(0, 10, (dst.numel(),), generator=gen)
    _, src_offsets = ref.group_by_source(src, 10)
    g = torch.randn(dst.numel(), 3, generator=gen, dtype=dtype)
    v = torch.randn(dst.numel(), 3, generator=gen, dtype=dtype)
    force, virial = ref.force_assembly_reference(g, v, src, dst, dst_offsets, src_offsets)
    e_force, e_virial = loops.force_assembly_loop(g, v, src, dst, 10)
    rtol = 1e-5 if dtype == torch.float32 else 1e-12
    assert_close_scaled(force, e_force, rtol=rtol, scale=rtol, what="force")
    assert_close_scaled(virial, e_virial, rtol=rtol, scale=rtol, what="virial")
    assert float(force.double().sum(0).abs().max()) <= (1e-5 if dtype == torch.float32 else 1e-12)


def test_gie_brute_force_and_shapes():
    gen = torch.Generator().manual_seed(3)
    dst = torch.randint(0, 6, (40,), generator=gen)
    zonal = torch.randn(40, 5, generator=gen)
    radial = torch.randn(40, 3, 4, generator=gen)
    slots = torch.tensor([0, 2, 2, 1, 0])
    inverse = torch.rand(6, generator=gen) + 0.2
    out = gie_ref.zonal_scatter_reference(zonal, radial, dst, slots, inverse)
    assert_close_scaled(out, loops.zonal_scatter_loop(zonal, radial, dst, slots, inverse), what="gie loop")
    torch.testing.assert_close(gie_ref.zonal_scatter_reference(zonal, radial, dst, slots, inverse.reshape(6, 1, 1)),
                               out, rtol=0, atol=0)
    empty = gie_ref.zonal_scatter_reference(torch.empty(0, 3), torch.empty(0, 2, 4), torch.empty(0, dtype=torch.int64),
                                            torch.tensor([0, 0, 1]), torch.ones(2))
    assert tuple(empty.shape) == (2, 4, 4) and int(empty.count_nonzero()) == 0
    with pytest.raises(ValueError, match="dst values"):
        gie_ref.zonal_scatter_reference(zonal, radial, dst + 6, slots, inverse)
    with pytest.raises(ValueError, match="radial_slot values"):
        gie_ref.zonal_scatter_reference(zonal, radial, dst, slots + 3, inverse)


@pytest.mark.parametrize("seed", range(3))
def test_gie_backward_brute_force(seed):
    gen = torch.Generator().manual_seed(40 + seed)
    nodes, edges, rows, radial_slots, channels = 7, 30, 6, 4, 3
    dst = torch.randint(0, nodes - 1, (edges,), generator=gen)  # the last node has no edge
    zonal = torch.randn(edges, rows, generator=gen)
    radial = torch.randn(edges, radial_slots, channels, generator=gen)
    slots = torch.randint(0, radial_slots - 1, (rows,), generator=gen)  # shared slots; the last one unreferenced
    inverse = torch.rand(nodes, generator=gen) + 0.2
    grad = torch.randn(nodes, rows + 1, channels, generator=gen)
    for shape in ((nodes,), (nodes, 1, 1)):
        got = gie_ref.zonal_scatter_backward_reference(grad, zonal, radial, dst, slots, inverse.reshape(shape))
        expected = loops.zonal_scatter_backward_loop(grad, zonal, radial, dst, slots, inverse.reshape(shape))
        for actual, truth, label in zip(got, expected, ("grad_zonal", "grad_radial", "grad_inv")):
            assert tuple(actual.shape) == truth.shape, label
            assert_close_scaled(actual, truth, what=label)
        assert int(got[1][:, radial_slots - 1].count_nonzero()) == 0, "unreferenced slot has a gradient"
        # row 0 of the output is 0 * inv: its cotangent reaches nothing
        shifted = grad.clone()
        shifted[:, 0] += 5.0
        again = gie_ref.zonal_scatter_backward_reference(shifted, zonal, radial, dst, slots, inverse.reshape(shape))
        for first, second in zip(got, again):
            torch.testing.assert_close(first, second, rtol=0, atol=0)


def test_rmsnorm_brute_force_and_backward_closed_form():
    gen = torch.Generator().manual_seed(9)
    x = torch.randn(4, 3, 33, generator=gen)
    scale = torch.rand(33, generator=gen) + 0.5
    out = rms_ref.rmsnorm(x, scale, 1e-6)
    assert_close_scaled(out, loops.rmsnorm_loop(x, scale, 1e-6), what="rmsnorm loop")
    g = torch.randn(x.shape, generator=gen)
    grad_x, grad_scale = rms_ref.rmsnorm_backward_reference(g, x, scale, 1e-6)
    xd, gd, sd = x.double().reshape(-1, 33), g.double().reshape(-1, 33), scale.double()
    inv = 1.0 / torch.sqrt((xd * xd).mean(1, keepdim=True) + 1e-6)
    u = gd * sd
    expected_x = inv * u - xd * inv ** 3 * (xd * u).mean(1, keepdim=True)
    assert_close_scaled(grad_x.reshape(-1, 33), expected_x, what="grad_x")
    assert_close_scaled(grad_scale, (gd * xd * inv).sum(0), what="grad_scale")
    for eps in (0.0, -1.0, float("inf"), float("nan")):
        with pytest.raises(ValueError, match="eps"):
            rms_ref.rmsnorm(x, scale, eps)


# ---------------------------------------------------------------------------
# 2b. the float64 closed forms the GPU gradient tests use as truth
# ---------------------------------------------------------------------------

def _assert_f64(actual, expected, what):
    assert_close_scaled(actual, expected, rtol=1e-12, scale=1e-12, what=what)


def test_closed_forms_against_golden_cases():
    for case in load_cases("segment_softmax"):
        alpha, null_alpha = closed_forms.segment_softmax_f64(case["logit"], case["env"], case["dst"],
                                                             case["offsets"].numel() - 1, case["null_logit"])
        _assert_f64(alpha, case["alpha_f64"], case["name"] + " alpha")
        if case["null_logit"] is not None:
            _assert_f64(null_alpha, case["null_alpha_f64"], case["name"] + " null_alpha")
    for case in load_cases("segment_softmax_backward"):
        gl, ge, gn = closed_forms.segment_softmax_backward_f64(case["grad_alpha"], case["logit"], case["env"],
                                                               case["dst"], case["offsets"].numel() - 1,
                                                               case["null_logit"], case["grad_null_alpha"])
        _assert_f64(gl, case["grad_logit_f64"], "grad_logit")
        _assert_f64(ge, case["grad_env_f64"], "grad_env")
        _assert_f64(gn, case["grad_null_logit_f64"], "grad_null")
    for case in load_cases("segment_sum_backward"):
        got = closed_forms.segment_sum_backward_f64(case["grad_out"], case["src"], case["dst"],
                                                    case["offsets"].numel() - 1, case["edge_scale"],
                                                    case["node_scale"])
        for actual, key in zip(got, ("grad_src_f64", "grad_edge_scale_f64", "grad_node_scale_f64")):
            _assert_f64(actual, case[key], key)
    for case in load_cases("zonal_scatter_backward"):
        got = closed_forms.zonal_scatter_backward_f64(case["grad_output"], case["zonal"], case["radial"],
                                                      case["dst"], case["radial_slot"], case["inv_sqrt_deg"])
        for actual, key in zip(got, ("grad_zonal_f64", "grad_radial_f64", "grad_inv_sqrt_deg_f64")):
            _assert_f64(actual, case[key], case["name"] + " " + key)


@pytest.mark.parametrize("seed", range(3))
def test_closed_forms_against_exact_loops_and_autograd(seed):
    logit, env, dst, offsets, null = _softmax_inputs(seed, masked_fraction=0.25)
    n_nodes = offsets.numel() - 1
    for with_null in (False, True):
        nl = null if with_null else None
        alpha, null_alpha = closed_forms.segment_softmax_f64(logit, env, dst, n_nodes, nl)
        e_alpha, e_null = loops.segment_softmax_loop(logit, env, dst, n_nodes, nl)
        _assert_f64(alpha, e_alpha, "alpha")
        if with_null:
            _assert_f64(null_alpha, e_null, "null alpha")
        # the closed-form backward against autograd of the float64 forward
        gen = torch.Generator().manual_seed(seed)
        ga = torch.randn(alpha.shape, generator=gen, dtype=torch.float64)
        gn = torch.randn((n_nodes, logit.shape[1]), generator=gen, dtype=torch.float64) if with_null else None
        leaves = [logit.double().requires_grad_(True), env.double().requires_grad_(True)]
        if with_null:
            leaves.append(null.double().requires_grad_(True))
        # the closed forms detach their inputs: autograd runs through a graph-keeping restatement
        a, na = _softmax_f64_differentiable(leaves[0], leaves[1], dst, n_nodes, leaves[2] if with_null else None)
        outs, cots = [a], [ga]
        if with_null:
            outs.append(na)
            cots.append(gn)
        auto = torch.autograd.grad(outs, leaves, cots)
        gl, ge, gnull = closed_forms.segment_softmax_backward_f64(ga, logit, env, dst, n_nodes, nl, gn)
        _assert_f64(gl, auto[0], "grad_logit vs autograd")
        _assert_f64(ge, auto[1], "grad_env vs autograd")
        if with_null:
            _assert_f64(gnull, auto[2], "grad_null vs autograd")

    gen = torch.Generator().manual_seed(60 + seed)
    nodes, edges, rows, radial_slots, channels = 6, 25, 5, 4, 3
    gdst = torch.randint(0, nodes, (edges,), generator=gen)
    zonal = torch.randn(edges, rows, generator=gen)
    radial = torch.randn(edges, radial_slots, channels, generator=gen)
    slots = torch.randint(0, radial_slots, (rows,), generator=gen)
    inverse = (torch.rand(nodes, generator=gen) + 0.2).reshape(nodes, 1, 1)
    grad = torch.randn(nodes, rows + 1, channels, generator=gen)
    got = closed_forms.zonal_scatter_backward_f64(grad, zonal, radial, gdst, slots, inverse)
    exact = loops.zonal_scatter_backward_loop(grad, zonal, radial, gdst, slots, inverse)
    for actual, truth, label in zip(got, exact, ("grad_zonal", "grad_radial", "grad_inv")):
        assert tuple(actual.shape) == truth.shape
        _assert_f64(actual, truth, label)

    sdst, soffsets = _random_graph(seed)
    sn = soffsets.numel() - 1
    src = torch.randn(sdst.numel(), 4, generator=gen)
    w = torch.rand(sdst.numel(), generator=gen) + 0.5
    s = torch.rand(sn, generator=gen) + 0.5
    g = torch.randn(sn, 4, generator=gen)
    leaves = [src.double().requires_grad_(True), w.double().requires_grad_(True), s.double().requires_grad_(True)]
    out = torch.zeros(sn, 4, dtype=torch.float64).index_add_(0, sdst, leaves[0] * leaves[1].reshape(-1, 1))
    out = out * leaves[2].reshape(-1, 1)
    auto = torch.autograd.grad(out, leaves, g.double())
    for actual, truth, label in zip(closed_forms.segment_sum_backward_f64(g, src, sdst, sn, w, s), auto,
                                    ("grad_src", "grad_w", "grad_s")):
        _assert_f64(actual, truth, label)

    x = torch.randn(3, 2, 19, generator=gen)
    scale = torch.rand(19, generator=gen) + 0.5
    g = torch.randn(x.shape, generator=gen)
    leaves = [x.double().requires_grad_(True), scale.double().requires_grad_(True)]
    y = leaves[0] / torch.sqrt(leaves[0].pow(2).mean(-1, keepdim=True) + 1e-6) * leaves[1]
    auto = torch.autograd.grad(y, leaves, g.double())
    gx, gs = closed_forms.rmsnorm_backward_f64(g, x, scale, 1e-6)
    _assert_f64(gx, auto[0], "rmsnorm grad_x")
    _assert_f64(gs, auto[1], "rmsnorm grad_scale")


def _softmax_f64_differentiable(logit, env, dst, n_nodes, null):
    valid = (env > 0).reshape(-1, 1)
    effective = torch.where(valid, logit + 2.0 * torch.log(env.clamp_min(1e-30)).reshape(-1, 1),
                            torch.full_like(logit, float("-inf")))
    peak = torch.full((n_nodes, logit.shape[1]), float("-inf"), dtype=torch.float64)
    peak = peak.scatter_reduce(0, dst.reshape(-1, 1).expand_as(logit), effective.detach(), reduce="amax")
    if null is not None:
        peak = torch.maximum(peak, null.detach())
    peak = torch.where(torch.isfinite(peak), peak, torch.zeros_like(peak))
    weight = torch.where(valid, torch.exp(effective - peak[dst]), torch.zeros_like(effective))
    null_weight = torch.exp(null - peak) if null is not None else torch.zeros_like(peak)
    total = torch.zeros_like(peak).index_add(0, dst, weight) + null_weight
    total = torch.where(total > 0, total, torch.ones_like(total))
    return weight / total[dst], (null_weight / total if null is not None else None)


# ---------------------------------------------------------------------------
# 3. planted mistakes: every check must reject a broken oracle
# ---------------------------------------------------------------------------

def _unstable_group(src, n_nodes):
    # ties broken by descending position: a plausible unstable sort
    keys = src * (src.numel() + 1) + (src.numel() - torch.arange(src.numel()))
    return torch.argsort(keys), ref.segment_offsets(src, n_nodes)


def _softmax_without_env(logit, env, dst, offsets, null_logit=None):
    return ref.segment_softmax_reference(logit, torch.where(env > 0, torch.ones_like(env), env), dst, offsets,
                                         null_logit)


def _softmax_single_log_env(logit, env, dst, offsets, null_logit=None):
    # ln(env) instead of 2 ln(env): env -> sqrt(env) halves the log term
    return ref.segment_softmax_reference(logit, torch.where(env > 0, env.clamp_min(1e-30).sqrt(), env), dst,
                                         offsets, null_logit)


def _softmax_null_out_of_denominator(logit, env, dst, offsets, null_logit=None):
    alpha, _ = ref.segment_softmax_reference(logit, env, dst, offsets, None)
    if null_logit is None:
        return alpha, None
    _, null_alpha = ref.segment_softmax_reference(logit, env, dst, offsets, null_logit)
    return alpha, null_alpha


def _force_wrong_sign(grad_edge, edge_vec, src, dst, dst_offsets, src_offsets):
    force, virial = ref.force_assembly_reference(grad_edge, edge_vec, src, dst, dst_offsets, src_offsets)
    # +g on the source side instead of -g
    return force + 2 * torch.zeros_like(force).index_add_(0, src, grad_edge), virial


def _force_transposed_virial(grad_edge, edge_vec, src, dst, dst_offsets, src_offsets):
    force, virial = ref.force_assembly_reference(grad_edge, edge_vec, src, dst, dst_offsets, src_offsets)
    return force, virial.reshape(-1, 3, 3).transpose(1, 2).reshape(-1, 9)


def _gie_normalise_first(zonal, radial, dst, radial_slot, inv_sqrt_deg):
    inverse = inv_sqrt_deg.reshape(-1)
    scaled = zonal * inverse[dst].reshape(-1, 1)
    return gie_ref.zonal_scatter_reference(scaled, radial, dst, radial_slot, torch.ones_like(inverse))


def _gie_wrong_slot(zonal, radial, dst, radial_slot, inv_sqrt_deg):
    return gie_ref.zonal_scatter_reference(zonal, radial, dst, torch.zeros_like(radial_slot), inv_sqrt_deg)


def _gie_backward_without_inverse(grad, zonal, radial, dst, radial_slot, inv_sqrt_deg):
    # grad_zonal taken from the unnormalised message: inv[n] dropped
    grad_zonal, grad_radial, grad_inv = gie_ref.zonal_scatter_backward_reference(grad, zonal, radial, dst,
                                                                                 radial_slot, inv_sqrt_deg)
    return grad_zonal / inv_sqrt_deg.reshape(-1)[dst].reshape(-1, 1), grad_radial, grad_inv


def _gie_backward_shared_slot_overwritten(grad, zonal, radial, dst, radial_slot, inv_sqrt_deg):
    # a scatter that assigns instead of accumulating: the last row sharing a slot wins
    grad_zonal, _, grad_inv = gie_ref.zonal_scatter_backward_reference(grad, zonal, radial, dst, radial_slot,
                                                                       inv_sqrt_deg)
    inverse = inv_sqrt_deg.reshape(-1)
    grad_radial = torch.zeros_like(radial)
    for r in range(zonal.shape[1]):
        grad_radial[:, int(radial_slot[r])] = (inverse[dst].reshape(-1, 1) * grad[dst, r + 1]
                                               * zonal[:, r].reshape(-1, 1))
    return grad_zonal, grad_radial, grad_inv


def _gie_backward_inverse_from_output(grad, zonal, radial, dst, radial_slot, inv_sqrt_deg):
    # grad_inv as the dot product with the normalised output instead of the pre-norm sum
    grad_zonal, grad_radial, _ = gie_ref.zonal_scatter_backward_reference(grad, zonal, radial, dst, radial_slot,
                                                                          inv_sqrt_deg)
    out = gie_ref.zonal_scatter_reference(zonal, radial, dst, radial_slot, inv_sqrt_deg)
    return grad_zonal, grad_radial, (grad * out).sum((1, 2)).reshape(inv_sqrt_deg.shape)


def _gie_backward_row_zero(grad, zonal, radial, dst, radial_slot, inv_sqrt_deg):
    # reading the cotangent of row r instead of row r + 1 (row 0 is the reserved one)
    shifted = torch.cat([grad[:, 1:], grad[:, :1]], dim=1)
    return gie_ref.zonal_scatter_backward_reference(shifted, zonal, radial, dst, radial_slot, inv_sqrt_deg)


def _edge_stream_coef_first(terms, activation=None, gate=None, gate_rows=None):
    moved = [(1.0, term[1] * float(term[0])) + tuple(term[2:]) for term in terms]
    return es_ref.edge_stream_combine_reference(moved, activation, gate, gate_rows)


def _edge_stream_gate_by_row(terms, activation=None, gate=None, gate_rows=None):
    if activation == "gate":
        gate_rows = [-1 if g < 0 else min(r, gate.shape[1] - 1) for r, g in enumerate(gate_rows)]
    return es_ref.edge_stream_combine_reference(terms, activation, gate, gate_rows)


def _edge_stream_silu_everywhere(terms, activation=None, gate=None, gate_rows=None):
    return es_ref.edge_stream_combine_reference(terms, "silu" if activation == "gate" else activation, gate, gate_rows)


def _rmsnorm_without_eps(x, scale=None, eps=1e-6):
    out = x * torch.rsqrt(x.square().mean(-1, keepdim=True))
    return out if scale is None else out * scale


def _rmsnorm_sum_not_mean(x, scale=None, eps=1e-6):
    out = x * torch.rsqrt(x.square().sum(-1, keepdim=True) + eps)
    return out if scale is None else out * scale


PLANTED = [
    ("unstable grouping", lambda: check_offsets(ref.segment_offsets, _unstable_group)),
    ("offsets off by one", lambda: check_offsets(lambda d, n: ref.segment_offsets(d, n) + 1, ref.group_by_source)),
    ("segment_sum drops node_scale",
     lambda: check_segment_sum(lambda s, d, o, w, n: ref.segment_sum_reference(s, d, o, w, None))),
    ("segment_sum drops edge_scale",
     lambda: check_segment_sum(lambda s, d, o, w, n: ref.segment_sum_reference(s, d, o, None, n))),
    ("segment_sum backward drops node_scale in grad_src",
     lambda: check_segment_sum_backward(
         lambda g, s, d, o, w, n: (lambda r: (r[0] / n[d].reshape(-1, 1), r[1], r[2]))(
             ref.segment_sum_backward_reference(g, s, d, o, w, n)))),
    ("softmax drops the envelope term", lambda: check_segment_softmax(_softmax_without_env)),
    ("softmax uses ln(env) instead of 2 ln(env)", lambda: check_segment_softmax(_softmax_single_log_env)),
    ("softmax leaves the null mass out of the denominator",
     lambda: check_segment_softmax(_softmax_null_out_of_denominator)),
    ("softmax backward drops the null term of S",
     lambda: check_segment_softmax_backward(
         lambda ga, l, e, d, o, n, gn: ref.segment_softmax_backward_reference(ga, l, e, d, o, n, torch.zeros_like(gn)))),
    ("force: wrong sign on the source side", lambda: check_force(_force_wrong_sign)),
    ("force: transposed virial", lambda: check_force(_force_transposed_virial)),
    ("gie normalises before the sum", lambda: check_gie(_gie_normalise_first)),
    ("gie ignores radial_slot", lambda: check_gie(_gie_wrong_slot)),
    ("gie backward drops inv in grad_zonal", lambda: check_gie_backward(_gie_backward_without_inverse)),
    ("gie backward overwrites a shared slot", lambda: check_gie_backward(_gie_backward_shared_slot_overwritten)),
    ("gie backward takes grad_inv from the output", lambda: check_gie_backward(_gie_backward_inverse_from_output)),
    ("gie backward reads the wrong cotangent row", lambda: check_gie_backward(_gie_backward_row_zero)),
    ("rmsnorm without eps", lambda: check_rmsnorm(_rmsnorm_without_eps)),
    ("rmsnorm with sum instead of mean", lambda: check_rmsnorm(_rmsnorm_sum_not_mean)),
    ("edge stream applies the coefficient before the product", lambda: check_edge_stream(_edge_stream_coef_first)),
    ("edge stream gates by row instead of gate_rows", lambda: check_edge_stream(_edge_stream_gate_by_row)),
    ("edge stream takes silu on the gated rows", lambda: check_edge_stream(_edge_stream_silu_everywhere)),
]


def test_edge_stream_oracle_pinned():
    check_edge_stream(es_ref.edge_stream_combine_reference)


@pytest.mark.parametrize("label,run", PLANTED, ids=[label for label, _ in PLANTED])
def test_planted_mistake_is_caught(label, run):
    with pytest.raises(AssertionError):
        run()
