"""The DeepMD seams with the real gfx950 operators (kernels.* -> libdpa4k.so) on cuda:0.

Each seam runs on a destination list that is grouped by segment but not
sorted (DeepMD's layout, so the CSR view carries an ``order``), and is compared
with DeepMD's stock path restated in tests/seam_fakes.py -- values and the
gradients that forces need (message, logits, envelope, source gate, bias).
Shapes follow the reference's opt-in parity test
(tests/csrc/accuracy/test_fused_deepmd_parity.py:45-110 of lipengfei1409/bysj).
"""
from __future__ import annotations

import pytest
import torch

from bysj_amd.model import fused_deepmd
from parity import announce, assert_close_scaled, assert_fp64, assert_gradient
from seam_fakes import FakeBlock, FakeModel, softmax_namespace, stock_softmax

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _shuffled_dst(n_nodes, n_edges, seed):
    gen = torch.Generator().manual_seed(seed)
    dst = torch.randint(0, n_nodes, (n_edges,), generator=gen)
    return dst.to(DEV)


@pytest.fixture
def clean():
    yield
    fused_deepmd.uninstall()


def test_softmax_seam_on_gfx950(clean):
    announce("seam softmax 512 nodes / 8192 edges / F*H = 16")
    space = softmax_namespace()
    stats = fused_deepmd.deepmd_patch(FakeModel([]), namespaces=[space], envelope=False, verbose=False)
    assert stats.bound_softmax, "the gfx950 operators should be usable on this device"
    gen = torch.Generator().manual_seed(1)
    dst = _shuffled_dst(512, 8192, seed=2)
    logits = (torch.randn(8192, 4, 4, generator=gen) * 2).to(DEV).requires_grad_(True)
    env = (torch.rand(8192, 1, generator=gen) + 0.05).to(DEV).requires_grad_(True)
    bias = torch.randn(4, 4, generator=gen).to(DEV).requires_grad_(True)
    upstream = torch.randn(8192, 4, 4, generator=gen).to(DEV)
    leaves = (logits, env, bias)
    alpha = space.segment_envelope_gated_softmax(logits, env, dst, 512, bias, 1e-6)
    grads = torch.autograd.grad(alpha, leaves, upstream)
    assert stats.softmax_hits == 1 and stats.softmax_fallbacks == 0, stats
    fused_deepmd.uninstall()
    expected = space.segment_envelope_gated_softmax(logits, env, dst, 512, bias, 1e-6)
    want = torch.autograd.grad(expected, leaves, upstream)
    # the stock path once more in float64 on the CPU: the truth both are held to
    leaves64 = tuple(t.detach().cpu().double().requires_grad_(True) for t in leaves)
    exact = stock_softmax(leaves64[0], leaves64[1], dst.cpu(), 512, leaves64[2], 1e-6)
    truth = torch.autograd.grad(exact, leaves64, upstream.cpu().double())
    assert_close_scaled(alpha, expected, what="alpha")
    assert_close_scaled(alpha, exact, what="alpha vs fp64 truth")
    for got, ref, exact_grad, name in zip(grads, want, truth, ("grad_logits", "grad_env", "grad_bias")):
        assert_gradient(got, ref, exact_grad, name)


@pytest.mark.parametrize("gate", [False, True])
def test_envelope_seam_on_gfx950(clean, gate):
    announce("seam envelope 64 nodes / 4096 edges / D=4 C=32", gate)
    gen = torch.Generator().manual_seed(3)
    n_nodes, n_edges = 64, 4096
    dst = _shuffled_dst(n_nodes, n_edges, seed=4)
    cache = type("EdgeCache", (), {})()
    cache.dst = dst
    cache.edge_env = (torch.rand(n_edges, 1, generator=gen) + 0.1).to(DEV).requires_grad_(True)
    cache.inv_sqrt_deg = torch.rsqrt(torch.bincount(dst.cpu(), minlength=n_nodes).float() + 1).reshape(-1, 1, 1).to(DEV)
    cache.edge_src_gate = (torch.rand(n_edges, 1, generator=gen) + 0.5).to(DEV).requires_grad_(True) if gate else None
    message = torch.randn(n_edges, 4, 32, generator=gen).to(DEV).requires_grad_(True)
    block = FakeBlock(message)
    stats = fused_deepmd.deepmd_patch(FakeModel([block]), softmax=False, verbose=False)
    assert stats.bound_envelope
    x = torch.zeros(n_nodes, 4, 32, device=DEV)
    upstream = torch.randn(n_nodes, 4, 32, generator=gen).to(DEV)
    leaves = (message, cache.edge_env) + ((cache.edge_src_gate,) if gate else ())
    out = block.forward_envelope(x, cache, None)
    grads = torch.autograd.grad(out, leaves, upstream)
    assert stats.envelope_hits == 1 and stats.envelope_fallbacks == 0, stats
    fused_deepmd.uninstall()
    expected = block.forward_envelope(x, cache, None)
    want = torch.autograd.grad(expected, leaves, upstream)
    # the stock path once more in float64 on the CPU: the truth both are held to
    leaves64 = tuple(t.detach().cpu().double().requires_grad_(True) for t in leaves)
    cache64 = type("EdgeCache", (), {})()
    cache64.dst = dst.cpu()
    cache64.edge_env = leaves64[1]
    cache64.inv_sqrt_deg = cache.inv_sqrt_deg.cpu().double()
    cache64.edge_src_gate = leaves64[2] if gate else None
    exact = FakeBlock(leaves64[0]).forward_envelope(x.cpu().double(), cache64, None)
    truth = torch.autograd.grad(exact, leaves64, upstream.cpu().double())
    assert_close_scaled(out, expected, what="aggregation")
    assert_close_scaled(out, exact, what="aggregation vs fp64 truth")
    for got, ref, exact_grad, name in zip(grads, want, truth, ("grad_message", "grad_edge_env", "grad_gate")):
        assert_gradient(got, ref, exact_grad, name)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_force_seam_on_gfx950_matches_the_stock_chain(clean, dtype):
    from seam_fakes import edge_force_virial_call, force_namespace

    announce("force seam", dtype)
    gen = torch.Generator().manual_seed(9)
    n_ext, n_edges = 500, 30000
    dst = torch.randint(0, n_ext, (n_edges,), generator=gen).to(DEV)  # unsorted extended-atom lists
    src = torch.randint(0, n_ext, (n_edges,), generator=gen).to(DEV)
    g = torch.randn(n_edges, 3, generator=gen, dtype=torch.float64).to(dtype).to(DEV)
    vec = torch.randn(n_edges, 3, generator=gen, dtype=torch.float64).to(dtype).to(DEV)
    space = force_namespace()
    stats = fused_deepmd.deepmd_patch(FakeModel([]), softmax=False, envelope=False, force=True,
                                      force_namespaces=[(space, "edge_force_virial")], verbose=False)
    args = edge_force_virial_call(g, vec, dst, src, n_ext)
    force, atom_virial, frame_virial, _ = space.edge_force_virial(*args)
    fused_deepmd.uninstall()
    stock = space.edge_force_virial(*args)
    assert stats.force_hits == 1 and stats.force_fallbacks == 0
    # the stock chain scatters with float atomics in the input dtype; the kernel accumulates in double:
    # both against the fp64 truth of the same sums
    g64, v64 = g.double().cpu(), vec.double().cpu()
    truth = force_namespace().edge_force_virial(*edge_force_virial_call(g64, v64, dst.cpu(), src.cpu(), n_ext))
    for label, got, exact, theirs in zip(("force", "atom virial", "frame virial"), (force, atom_virial, frame_virial),
                                         truth, stock):
        if dtype == torch.float64:
            assert_fp64(got, exact, f"{label} vs fp64 truth")
        else:
            assert_close_scaled(got, exact, what=f"{label} vs fp64 truth")
            assert_close_scaled(got, theirs, what=f"{label} vs the stock chain")


def test_force_seam_builds_the_blob_plan_once_per_graph(clean, monkeypatch):
    """A water graph above the plan threshold, in a shuffled natural edge order (DeepMD's extended lists): two
    seam calls with fresh per-edge gradients build one blob plan, run the planned kernels both times, and
    match the stock chain."""
    from bysj_amd import workloads
    from bysj_amd.kernels import _C
    from bysj_amd.kernels import segment as segment_ops
    from seam_fakes import edge_force_virial_call, force_namespace

    graph = workloads.water_graph(2048, seed=4)
    n_edges = graph.n_edges
    assert n_edges >= segment_ops._ForcePlanCache.MIN_EDGES
    announce("force seam plan reuse", 2048, n_edges)
    shuffle = torch.randperm(n_edges, generator=torch.Generator().manual_seed(5))
    dst = torch.from_numpy(graph.dst)[shuffle].to(DEV)
    src = torch.from_numpy(graph.src)[shuffle].to(DEV)
    vec = torch.from_numpy(graph.edge_vec)[shuffle].float().contiguous().to(DEV)
    builds, planned = [], []
    build = _C.force_assembly_plan
    run = _C.force_assembly

    def counting_build(*args, **kwargs):
        builds.append(args[2])
        return build(*args, **kwargs)

    def recording_run(*args, plan=None):
        planned.append(plan is not None)
        return run(*args, plan=plan)

    monkeypatch.setattr(_C, "force_assembly_plan", counting_build)
    monkeypatch.setattr(_C, "force_assembly", recording_run)
    segment_ops._FORCE_PLANS.clear()
    space = force_namespace()
    stats = fused_deepmd.deepmd_patch(FakeModel([]), softmax=False, envelope=False, force=True,
                                      force_namespaces=[(space, "edge_force_virial")], verbose=False)
    gen = torch.Generator().manual_seed(6)
    g0 = torch.randn(n_edges, 3, generator=gen).to(DEV)
    args = list(edge_force_virial_call(g0, vec, dst, src, 2048))
    results = []
    for step in range(2):
        args[0] = torch.randn(n_edges, 3, generator=gen).to(DEV) if step else g0  # new gradients each step
        results.append((tuple(args), space.edge_force_virial(*args)))
    assert stats.force_hits == 2 and stats.force_fallbacks == 0, stats
    assert len(builds) == 1, f"one blob plan per graph, got {len(builds)} builds"
    assert planned == [True, True], "both calls run the planned kernels"
    fused_deepmd.uninstall()
    for call_args, (force, atom_virial, frame_virial, _) in results:
        stock = space.edge_force_virial(*call_args)
        for label, got, theirs in zip(("force", "atom virial", "frame virial"), (force, atom_virial, frame_virial),
                                      stock):
            assert_close_scaled(got, theirs, what=f"{label} vs the stock chain")
    segment_ops._FORCE_PLANS.clear()
