"""The planned (bucketed two-pass) force assembly against the direct gather kernel.

The planned path (dpa4k_force_assembly_plan + dpa4k_force_assembly_f*_planned)
accumulates in the direct kernel's order, so the two must agree bit for bit;
the direct kernel is itself checked against the oracle and an fp64 truth in
test_gpu_segment.py, and one case here repeats that check.  The plan's layout
is checked exactly against a NumPy restatement: the edges sorted stably by
(tile of 8192 edges, source bucket), and each source slot's row in that order.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from bysj_amd import workloads
from bysj_amd.kernels import _C
from oracle import loops
from oracle import segment as ref
from parity import announce, assert_bitwise, assert_close_scaled, assert_fp64

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
TILE, MOST_BUCKETS = 8192, 256


def _random_graph(atoms, edges, seed, hubs=()):
    gen = torch.Generator().manual_seed(seed)
    dst = torch.sort(torch.randint(0, atoms, (edges,), generator=gen)).values
    src = torch.randint(0, atoms, (edges,), generator=gen)
    for hub, count in hubs:  # atoms that are the source of many edges
        picks = torch.randperm(edges, generator=gen)[:count]
        src[picks] = hub
    g = torch.randn(edges, 3, generator=gen, dtype=torch.float64)
    v = torch.randn(edges, 3, generator=gen, dtype=torch.float64)
    order, src_offsets = ref.group_by_source(src, atoms)
    return {"grad_edge": g, "edge_vec": v, "src": src, "dst": dst, "dst_offsets": ref.segment_offsets(dst, atoms),
            "src_offsets": src_offsets, "src_order": order}


def _water(atoms, seed, spatial):
    graph = workloads.water_graph(atoms, seed=seed, spatial_order=spatial)
    return workloads.force_config(graph, seed=seed, device="cpu", dtype=torch.float64)


CASES = {
    "water_random_numbering": lambda: _water(4096, 5, False),
    "water_morton_numbering": lambda: _water(4096, 5, True),
    "source_hubs": lambda: _random_graph(700, 20000, 11, hubs=((3, 600), (650, 250))),
    "three_atoms": lambda: _random_graph(3, 5, 12),
    "one_tile_and_one_edge": lambda: _random_graph(300, TILE * 2 + 1, 13),
}


def _decode_plan(plan: _C.ForcePlan, edges: int):
    """edge_row and src_pos from the plan buffer (two int32 arrays, 256-byte aligned)."""
    stride = -(-4 * max(edges, 1) // 256) * 256
    raw = plan.buffer.cpu().numpy()
    return [raw[i * stride:i * stride + 4 * edges].view(np.int32) for i in range(2)]


def _expected_slots(case, atoms):
    """Edges sorted stably by (tile of 8192 edges, bucket of their source atom)."""
    edges = case["src_order"].numel()
    wanted = min(atoms, MOST_BUCKETS)
    bucket_atoms = -(-atoms // wanted)
    buckets = -(-atoms // bucket_atoms)
    src_of = np.zeros(edges, dtype=np.int64)  # edges no valid slot names keep bucket 0
    offsets, order = case["src_offsets"].numpy(), case["src_order"].numpy()
    for atom in range(atoms):
        slots = order[offsets[atom]:offsets[atom + 1]]
        valid = slots[(slots >= 0) & (slots < edges)]
        src_of[valid] = atom
    key = (np.arange(edges) // TILE) * buckets + src_of // bucket_atoms
    return np.argsort(key, kind="stable")


def _check_plan_layout(plan, case, atoms):
    edges = case["src_order"].numel()
    edge_row, src_pos = _decode_plan(plan, edges)
    position = np.empty(edges, dtype=np.int64)
    position[_expected_slots(case, atoms)] = np.arange(edges)
    np.testing.assert_array_equal(edge_row, position, err_msg="plan: row of each edge")
    order = case["src_order"].numpy()
    valid = (order >= 0) & (order < edges)
    expected = np.where(valid, position[np.clip(order, 0, max(edges - 1, 0))], -1)
    np.testing.assert_array_equal(src_pos, expected, err_msg="plan: source positions")


def _run(case, dtype, plan=None):
    d = {k: v.to(DEV) for k, v in case.items()}
    return _C.force_assembly(d["grad_edge"].to(dtype), d["edge_vec"].to(dtype), d["dst_offsets"], d["src_offsets"],
                             d["src_order"], plan=plan)


@pytest.mark.parametrize("name", list(CASES))
def test_planned_force_matches_the_direct_kernel_bit_for_bit(name):
    case = CASES[name]()
    atoms = case["dst_offsets"].numel() - 1
    announce("force plan", name, atoms, case["src_order"].numel())
    plan8 = _C.force_assembly_plan(case["src_offsets"].to(DEV), case["src_order"].to(DEV), value_bytes=8)
    plan4 = _C.force_assembly_plan(case["src_offsets"].to(DEV), case["src_order"].to(DEV), value_bytes=4)
    _check_plan_layout(plan8, case, atoms)
    for dtype, plans in ((torch.float32, (plan8, plan4)), (torch.float64, (plan8,))):
        direct = _run(case, dtype)
        for plan in plans:
            planned = _run(case, dtype, plan)
            again = _run(case, dtype, plan)
            for label, a, b, c in zip(("force", "virial"), direct, planned, again):
                assert_bitwise(b, a, f"{name} {dtype} {label}: planned vs direct (plan of {plan.value_bytes} bytes)")
                assert_bitwise(c, b, f"{name} {dtype} {label}: planned run to run")


def test_planned_force_against_the_oracle_and_truth():
    case = _random_graph(500, 30000, 17, hubs=((7, 400),))
    announce("force plan vs oracle")
    plan = _C.force_assembly_plan(case["src_offsets"].to(DEV), case["src_order"].to(DEV))
    force, virial = _run(case, torch.float32, plan)
    g, v = case["grad_edge"].float(), case["edge_vec"].float()
    e_force, e_virial = ref.force_assembly_reference(g, v, case["src"], case["dst"], case["dst_offsets"],
                                                     case["src_offsets"])
    t_force, t_virial = loops.force_assembly_loop(g, v, case["src"], case["dst"], 500)
    assert_close_scaled(force, e_force, what="fp32 force vs oracle")
    assert_close_scaled(virial, e_virial, what="fp32 virial vs oracle")
    assert_close_scaled(force, t_force, what="fp32 force vs truth")
    assert_close_scaled(virial, t_virial, what="fp32 virial vs truth")
    force64, virial64 = _run(case, torch.float64, plan)
    t_force, t_virial = loops.force_assembly_loop(case["grad_edge"], case["edge_vec"], case["src"], case["dst"], 500)
    assert_fp64(force64, t_force, "fp64 force vs truth")
    assert_fp64(virial64, t_virial, "fp64 virial vs truth")


def test_planned_force_skips_invalid_source_slots_like_the_direct_kernel():
    case = _random_graph(200, 9000, 19)
    order = case["src_order"].clone()
    order[5], order[700], order[-1] = -1, order.numel() + 7, -3
    case["src_order"] = order
    announce("force plan, invalid slots")
    plan = _C.force_assembly_plan(case["src_offsets"].to(DEV), order.to(DEV))
    _check_plan_layout(plan, case, 200)
    for dtype in (torch.float32, torch.float64):
        for label, a, b in zip(("force", "virial"), _run(case, dtype), _run(case, dtype, plan)):
            assert_bitwise(b, a, f"{dtype} {label} with invalid slots")


def test_planned_force_without_edges_and_plan_checks():
    announce("force plan, empty graph and checks")
    offsets = torch.zeros(5, dtype=torch.int64, device=DEV)
    order = torch.empty(0, dtype=torch.int64, device=DEV)
    empty = torch.empty((0, 3), device=DEV)
    plan = _C.force_assembly_plan(offsets, order, value_bytes=4)
    force, virial = _C.force_assembly(empty, empty, offsets, offsets, order, plan=plan)
    assert force.shape == (4, 3) and virial.shape == (4, 9)
    assert force.count_nonzero().item() == 0 and virial.count_nonzero().item() == 0
    case = _random_graph(50, 800, 23)
    plan = _C.force_assembly_plan(case["src_offsets"].to(DEV), case["src_order"].to(DEV), value_bytes=4)
    with pytest.raises(RuntimeError, match="another graph, device or dtype"):
        _run(case, torch.float64, plan)  # a float32 plan cannot hold float64 rows
    other = _random_graph(50, 801, 23)
    with pytest.raises(RuntimeError, match="another graph"):
        _run(other, torch.float32, plan)


def test_operator_plans_float32_on_scattered_numbering_only():
    """kernels.force_assembly builds a plan for float32 on a graph without spatial locality, and for no other."""
    from bysj_amd import kernels
    from bysj_amd.kernels import segment as segment_ops

    announce("force plan policy")
    segment_ops._FORCE_PLANS.clear()
    results = {}
    for spatial in (False, True):
        # 16,384 atoms (1.5M edges): with random numbering an atom's source edges lie ~16K edges apart
        case = _water(16384, 6, spatial)
        assert case["src_order"].numel() >= segment_ops._ForcePlanCache.MIN_EDGES
        d = {k: v.to(DEV) for k, v in case.items()}
        args = (d["grad_edge"].float(), d["edge_vec"].float(), d["src"], d["dst"], d["dst_offsets"],
                d["src_offsets"], d["src_order"])
        force, virial = kernels.force_assembly(*args)
        entry = segment_ops._FORCE_PLANS._entries[id(d["src_order"])]
        assert (entry[2] is not None) == (not spatial), "a plan exactly for the scattered numbering"
        direct = _C.force_assembly(args[0], args[1], d["dst_offsets"], d["src_offsets"], d["src_order"])
        assert_bitwise(force, direct[0], f"operator force (spatial={spatial})")
        assert_bitwise(virial, direct[1], f"operator virial (spatial={spatial})")
        # float64 calls never build or use a plan
        force64, _ = kernels.force_assembly(d["grad_edge"], d["edge_vec"], d["src"], d["dst"], d["dst_offsets"],
                                            d["src_offsets"], d["src_order"])
        assert force64.dtype == torch.float64
        results[spatial] = d
    # an in-place write to src_order drops the cached plan; the next call measures and plans again
    d = results[False]
    before = segment_ops._FORCE_PLANS._entries[id(d["src_order"])][2]
    d["src_order"].add_(0)
    kernels.force_assembly(d["grad_edge"].float(), d["edge_vec"].float(), d["src"], d["dst"], d["dst_offsets"],
                           d["src_offsets"], d["src_order"])
    after = segment_ops._FORCE_PLANS._entries[id(d["src_order"])][2]
    assert after is not None and after is not before
    segment_ops._FORCE_PLANS.clear()
