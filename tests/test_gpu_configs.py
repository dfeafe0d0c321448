"""Configurations 3 and 4 at their full sizes, on their own water-box workloads.

BASELINE.json config 3 (GIE zonal scatter then RMSNorm, N = 24,576 atoms,
~2.2M edges, [E, 16, 64] features) and config 4 (force assembly in fp32 and
fp64, N = 65,536 atoms, ~5.9M edges) run here exactly as bench.py generates
them (workloads.water_graph, seed 0).  The full outputs are too large for the
CPU oracle, so sampled atoms -- the first, the last and random ones -- are
checked against it on the sub-graph of the edges they own (an atom's outputs
depend only on its own edges, so the sub-graph gives the oracle the same
terms), against an fp64 truth, and through size-independent properties over
the whole output: Newton's third law, run-to-run bitwise reproducibility, and
for config 3 the fused kernel against the two operators bit for bit.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from bysj_amd import kernels, workloads
from bysj_amd.kernels import gie as gie_ops
from closed_forms import gie_rmsnorm_chain_f64
from oracle import gie as gie_ref
from oracle import loops
from oracle import segment as ref
from oracle.rmsnorm import rmsnorm as rmsnorm_ref
from parity import announce, assert_bitwise, assert_close_scaled, assert_fp64, assert_gradient

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


@pytest.fixture(autouse=True)
def _release():
    yield
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def _samples(n: int, seed: int, count: int = 20) -> np.ndarray:
    picks = {0, 1, n - 2, n - 1}
    picks.update(workloads.rng(seed).integers(0, n, size=count).tolist())
    return np.array(sorted(picks), dtype=np.int64)


# ---------------------------------------------------------------------------
# config 4: force assembly, N = 65,536
# ---------------------------------------------------------------------------

def _force_subgraph(graph: workloads.WaterGraph, atoms: np.ndarray):
    """Edges whose destination or source is a sampled atom (natural order kept, so still
    destination-grouped), with the atoms they touch renumbered 0..U-1 in ascending order."""
    sampled = np.zeros(graph.n_atoms, dtype=bool)
    sampled[atoms] = True
    edges = np.nonzero(sampled[graph.dst] | sampled[graph.src])[0]
    touched = np.unique(np.concatenate([graph.dst[edges], graph.src[edges], atoms]))
    renumber = np.full(graph.n_atoms, -1, dtype=np.int64)
    renumber[touched] = np.arange(touched.size)
    return edges, touched.size, renumber[graph.dst[edges]], renumber[graph.src[edges]], renumber[atoms]


@pytest.mark.parametrize("spatial_order", [False, True], ids=["random_numbering", "morton_numbering"])
def test_force_assembly_config4_full_size(spatial_order):
    announce("config 4 force, 65536 atoms", "morton" if spatial_order else "random")
    graph = workloads.water_graph(65536, seed=0, spatial_order=spatial_order, device=DEV)
    atoms = _samples(graph.n_atoms, seed=4)
    edges, n_sub, sub_dst, sub_src, sub_atoms = _force_subgraph(graph, atoms)
    sub_dst_t, sub_src_t = torch.from_numpy(sub_dst), torch.from_numpy(sub_src)
    dst_offsets = ref.segment_offsets(sub_dst_t, n_sub)
    src_offsets = ref.segment_offsets(sub_src_t, n_sub)
    for dtype in (torch.float32, torch.float64):
        case = workloads.force_config(graph, seed=0, device=DEV, dtype=dtype)
        args = (case["grad_edge"], case["edge_vec"], case["src"], case["dst"], case["dst_offsets"],
                case["src_offsets"], case["src_order"])
        force, virial = kernels.force_assembly(*args)
        again_force, again_virial = kernels.force_assembly(*args)
        assert_bitwise(again_force, force, f"{dtype} force run to run")
        assert_bitwise(again_virial, virial, f"{dtype} virial run to run")

        # Newton's third law over all atoms: every edge adds +g and -g, so the exact total is zero.
        # fp64 keeps the reference's rule; fp32 outputs are each rounded once from a double sum, so
        # the total of the rounded values is bounded by the sum of their half-ulp rounding errors.
        total = force.double().sum(0).abs().max().item()
        if dtype == torch.float64:
            assert total <= 1e-12 * case["grad_edge"].abs().sum().item(), total
        else:
            bound = force.double().abs().sum(0).max().item() * 2.0 ** -24
            assert total <= bound, (total, bound)

        index = torch.from_numpy(edges).to(DEV)
        g = case["grad_edge"].index_select(0, index).cpu()
        v = case["edge_vec"].index_select(0, index).cpu()
        e_force, e_virial = ref.force_assembly_reference(g, v, sub_src_t, sub_dst_t, dst_offsets, src_offsets)
        t_force, t_virial = loops.force_assembly_loop(g, v, sub_src_t, sub_dst_t, n_sub)
        got_force = force.index_select(0, torch.from_numpy(atoms).to(DEV)).cpu()
        got_virial = virial.index_select(0, torch.from_numpy(atoms).to(DEV)).cpu()
        pick = torch.from_numpy(sub_atoms)
        if dtype == torch.float64:
            assert_fp64(got_force, e_force[pick], "fp64 force vs oracle")
            assert_fp64(got_virial, e_virial[pick], "fp64 virial vs oracle")
            assert_fp64(got_force, t_force[sub_atoms], "fp64 force vs exact sum")
            assert_fp64(got_virial, t_virial[sub_atoms], "fp64 virial vs exact sum")
        else:
            assert_close_scaled(got_force, e_force[pick], what="fp32 force vs oracle")
            assert_close_scaled(got_virial, e_virial[pick], what="fp32 virial vs oracle")
            assert_close_scaled(got_force, t_force[sub_atoms], what="fp32 force vs exact sum")
            assert_close_scaled(got_virial, t_virial[sub_atoms], what="fp32 virial vs exact sum")
        del case, force, virial, again_force, again_virial


# ---------------------------------------------------------------------------
# config 3: GIE zonal scatter -> RMSNorm, N = 24,576
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("primary", [True, False], ids=["radial_16_slots", "radial_3_slots_deepmd"])
def test_gie_rmsnorm_config3_full_size(primary):
    announce("config 3 gie -> rmsnorm, 24576 atoms", "primary" if primary else "secondary")
    graph = workloads.water_graph(24576, seed=0, device=DEV)
    case = workloads.gie_config(graph, seed=0, device=DEV, primary=primary)
    n_atoms, width = graph.n_atoms, 16 * 64
    z = case["zonal"].requires_grad_(True)
    r = case["radial"].requires_grad_(True)
    inv = case["inv_sqrt_deg"].clone().requires_grad_(True)
    scale = case["rms_scale"].clone().requires_grad_(True)
    x = kernels.zonal_scatter(z, r, case["dst"], case["radial_slot"], inv)
    y = kernels.rmsnorm(x.reshape(n_atoms, width), scale, eps=1e-6)
    with torch.no_grad():
        fused = gie_ops.gie_zonal_scatter_rmsnorm(case["zonal"], case["radial"], case["dst"], case["radial_slot"],
                                                  case["inv_sqrt_deg"], scale=case["rms_scale"], eps=1e-6)
        again = kernels.zonal_scatter(case["zonal"], case["radial"], case["dst"], case["radial_slot"],
                                      case["inv_sqrt_deg"])
    assert_bitwise(fused.reshape(n_atoms, width), y, "fused GIE -> RMSNorm vs the two operators")
    assert_bitwise(again, x, "GIE run to run")
    del fused, again
    generator = torch.Generator(device=DEV)
    generator.manual_seed(31)
    up = torch.randn((n_atoms, width), generator=generator, device=DEV)
    grads = torch.autograd.grad(y, (z, r, inv, scale), up)

    atoms = _samples(n_atoms, seed=3)
    offsets = graph.offsets()
    edges = np.concatenate([np.arange(offsets[a], offsets[a + 1]) for a in atoms])
    sub_dst = torch.from_numpy(np.repeat(np.arange(atoms.size), offsets[atoms + 1] - offsets[atoms]))
    edge_index, atom_index = torch.from_numpy(edges).to(DEV), torch.from_numpy(atoms).to(DEV)
    inputs = (case["zonal"].detach().index_select(0, edge_index).cpu(),
              case["radial"].detach().index_select(0, edge_index).cpu(), sub_dst, case["radial_slot"].cpu(),
              case["inv_sqrt_deg"].index_select(0, atom_index).cpu())
    expected_x = gie_ref.zonal_scatter_reference(*inputs).reshape(atoms.size, width)
    assert_bitwise(x.detach().reshape(n_atoms, width).index_select(0, atom_index), expected_x,
                   "GIE rows of the sampled atoms vs oracle")
    expected_y = rmsnorm_ref(expected_x, case["rms_scale"].cpu(), 1e-6)
    got_y = y.detach().index_select(0, atom_index).cpu()
    assert_close_scaled(got_y, expected_y, what="RMSNorm rows vs oracle")
    assert_close_scaled(got_y, loops.rmsnorm_loop(expected_x, case["rms_scale"].cpu(), 1e-6),
                        what="RMSNorm rows vs fp64 truth")

    # gradients of the sampled atoms' edges and inverse degrees: the oracle chain and the fp64 chain
    sub_up = up.index_select(0, atom_index).cpu()
    leaves = [inputs[0].clone().requires_grad_(True), inputs[1].clone().requires_grad_(True),
              inputs[4].clone().requires_grad_(True)]
    oracle_y = rmsnorm_ref(gie_ref.zonal_scatter_reference(leaves[0], leaves[1], sub_dst, inputs[3], leaves[2])
                           .reshape(atoms.size, width), case["rms_scale"].cpu(), 1e-6)
    oracle = torch.autograd.grad(oracle_y, leaves, sub_up)
    truth, terms = gie_rmsnorm_chain_f64(inputs, case["rms_scale"], sub_up.reshape(atoms.size, 16, 64), 1e-6)
    got_zonal = grads[0].index_select(0, edge_index).cpu()
    got_radial = grads[1].index_select(0, edge_index).cpu()
    got_inv = grads[2].index_select(0, atom_index).cpu()
    assert_gradient(got_zonal, oracle[0], truth[0], "grad zonal")
    assert_gradient(got_radial, oracle[1], truth[1], "grad radial")
    # the inverse degree's gradient is a sum of terms that cancel (RMSNorm is scale invariant):
    # held to 1e-5 of the sum of its terms' sizes, as in the reduced-size test
    error = (got_inv.double() - truth[2]).abs()
    assert bool((error <= 1e-5 * terms + 1e-12).all()), f"grad inverse: worst {float((error / terms).max())}"
    # the scale's gradient sums over every row: against the fp64 closed form sum_rows up * x * inv_rms,
    # evaluated on the device from the verified GIE rows
    x64 = x.detach().reshape(n_atoms, width).double()
    inv_rms = torch.rsqrt(x64.square().mean(1, keepdim=True) + 1e-6)
    expected_scale = (up.double() * x64 * inv_rms).sum(0)
    assert_close_scaled(grads[3], expected_scale, what="grad scale vs fp64 closed form")
