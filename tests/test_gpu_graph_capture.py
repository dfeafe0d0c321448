"""The operators under HIP graph capture: every replay equals the eager result.

The library clears memory with a fill kernel rather than hipMemsetAsync and
does not synchronise inside an operator, so a caller may capture forward and
backward passes in a HIP graph.  What synchronises -- the CSR builders, the
GIE grouping and the softmax degree plan -- runs once per graph before
capture: kernels.segment_softmax and kernels.zonal_scatter cache the plan
and the grouping per tensor, so a call captured after one eager call on the
same tensors replays without them.  Each case captures a step (forward and
gradients), then three times writes new input values in place, does other
eager work, synchronises, replays, and compares every output bit for bit
with an eager step on the same inputs.
"""
from __future__ import annotations

import pytest
import torch

from bysj_amd import kernels, workloads
from bysj_amd.kernels.gie import gie_zonal_scatter_rmsnorm
from parity import announce, assert_bitwise

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
REPLAYS = 3


def _csr(n_nodes, mean, seed, hubs=0, hub_degree=0):
    degrees = workloads.poisson_degrees(n_nodes, mean, seed, minimum=0)
    if hubs:
        degrees[workloads.rng(seed + 1).choice(n_nodes, size=hubs, replace=False)] = hub_degree
    offsets = torch.from_numpy(workloads.offsets_from_degrees(degrees)).to(DEV)
    dst = torch.from_numpy(workloads.dst_from_degrees(degrees)).to(DEV)
    return dst, offsets


def _check_replays(step, leaves, seed):
    """Capture step(); before each replay refill `leaves` in place and compare with eager."""
    gen = torch.Generator(device=DEV)
    gen.manual_seed(seed)
    for _ in range(2):  # warm up (builds plans and groupings) on a side stream, as capture expects
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            step()
        torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = step()
    for replay in range(REPLAYS):
        with torch.no_grad():
            for leaf in leaves:
                fresh = torch.rand(leaf.shape, generator=gen, device=DEV, dtype=leaf.dtype) + 0.25
                leaf.copy_(fresh)
        noise = torch.randn(1 << 20, device=DEV, generator=gen).cumsum(0)  # unrelated eager work
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        expected = step()
        torch.cuda.synchronize()
        for i, (got, want) in enumerate(zip(captured, expected)):
            assert_bitwise(got, want, f"replay {replay} output {i}")
        del noise


def _grads(outputs, inputs, cotangents):
    return torch.autograd.grad(outputs, inputs, cotangents)


def test_segment_sum_capture():
    announce("capture segment_sum")
    dst, offsets = _csr(3000, 20, seed=1)
    edges = dst.numel()
    src = torch.rand(edges, 64, device=DEV, requires_grad=True)
    w = torch.rand(edges, device=DEV, requires_grad=True)
    s = torch.rand(3000, device=DEV, requires_grad=True)
    grad = torch.randn(3000, 64, device=DEV)

    def step():
        out = kernels.segment_sum(src, dst, offsets, w, s)
        return (out.detach(),) + _grads(out, (src, w, s), grad)

    _check_replays(step, (src, w, s), seed=1)


@pytest.mark.parametrize("channels", [8, 64])
def test_segment_softmax_capture(channels):
    announce("capture segment_softmax", channels)
    dst, offsets = _csr(4000, 12, seed=2, hubs=8, hub_degree=400)
    edges = dst.numel()
    logit = torch.rand(edges, channels, device=DEV, requires_grad=True)
    env = torch.rand(edges, device=DEV, requires_grad=True)
    null = torch.rand(4000, channels, device=DEV, requires_grad=True)
    cot = (torch.randn(edges, channels, device=DEV), torch.randn(4000, channels, device=DEV))

    def step():
        alpha, null_alpha = kernels.segment_softmax(logit, env, offsets, null)
        return (alpha.detach(), null_alpha.detach()) + _grads((alpha, null_alpha), (logit, env, null), cot)

    _check_replays(step, (logit, env, null), seed=2)


@pytest.mark.parametrize("fused", [False, True])
def test_gie_capture(fused):
    announce("capture gie", fused)
    n_nodes, channels = 1500, 16
    dst, _ = _csr(n_nodes, 9, seed=3)
    edges = dst.numel()
    dst = dst[torch.randperm(edges, device=DEV)]  # unsorted: the grouping has an order
    slots = torch.arange(1, 16, dtype=torch.int64, device=DEV)
    zonal = torch.rand(edges, 15, device=DEV, requires_grad=True)
    radial = torch.rand(edges, 16, channels, device=DEV, requires_grad=True)
    inv = torch.rand(n_nodes, device=DEV, requires_grad=True)
    scale = torch.rand(16 * channels, device=DEV, requires_grad=True)
    grad = torch.randn(n_nodes, 16, channels, device=DEV)

    def step():
        if fused:
            out = gie_zonal_scatter_rmsnorm(zonal, radial, dst, slots, inv, scale)
            inputs = (zonal, radial, inv, scale)
        else:
            out = kernels.zonal_scatter(zonal, radial, dst, slots, inv)
            inputs = (zonal, radial, inv)
        return (out.detach(),) + _grads(out, inputs, grad)

    _check_replays(step, (zonal, radial, inv, scale), seed=3)


@pytest.mark.parametrize("width", [1024, 8200])
def test_rmsnorm_capture(width):
    announce("capture rmsnorm", width)
    x = torch.rand(2000, width, device=DEV, requires_grad=True)
    scale = torch.rand(width, device=DEV, requires_grad=True)
    grad = torch.randn(2000, width, device=DEV)

    def step():
        y = kernels.rmsnorm(x, scale)
        return (y.detach(),) + _grads(y, (x, scale), grad)

    _check_replays(step, (x, scale), seed=4)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_force_assembly_capture(dtype):
    announce("capture force_assembly", dtype)
    dst, dst_offsets = _csr(3000, 25, seed=5)
    edges = dst.numel()
    src = torch.randint(0, 3000, (edges,), device=DEV)
    src_order, src_offsets = kernels.group_by_source(src, 3000)  # synchronises: before capture
    grad_edge = torch.rand(edges, 3, device=DEV, dtype=dtype)
    edge_vec = torch.rand(edges, 3, device=DEV, dtype=dtype)

    def step():
        return kernels.force_assembly(grad_edge, edge_vec, src, dst, dst_offsets, src_offsets, src_order)

    _check_replays(step, (grad_edge, edge_vec), seed=5)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_force_assembly_planned_capture(dtype):
    """A water graph keeps its blob plan (built by the first eager call), so the planned passes are
    what the graph records.  16,384 atoms: with random numbering an atom's source edges lie far apart
    (about 16K edges), so float64 is planned too."""
    from bysj_amd.kernels import segment as segment_ops

    announce("capture planned force_assembly", dtype)
    graph = workloads.water_graph(16384, seed=7, device=DEV)
    case = workloads.force_config(graph, seed=7, device=DEV, dtype=dtype)
    grad_edge, edge_vec = case["grad_edge"], case["edge_vec"]

    def step():
        return kernels.force_assembly(grad_edge, edge_vec, case["src"], case["dst"], case["dst_offsets"],
                                      case["src_offsets"], case["src_order"])

    step()  # builds the plan outside the capture
    assert segment_ops._FORCE_PLANS._entries[(id(case["src_order"]), dtype)][2] is not None
    _check_replays(step, (grad_edge,), seed=7)


@pytest.mark.parametrize("activation", [None, "gate"])
def test_edge_stream_capture(activation):
    from bysj_amd.kernels import edge_stream

    announce("capture edge_stream", activation)
    x = torch.rand(2000, 9, 64, device=DEV)
    a = torch.rand(2000, 9, 64, device=DEV)
    s = torch.rand(2000, 9, 1, device=DEV)
    q = torch.rand(2000, 2, 64, device=DEV)
    rows = [-1, 0, 0, 0, 1, 1, 1, 1, 1]
    acc = torch.empty(2000, 9, 64, device=DEV)

    def step():
        with torch.no_grad():
            out = edge_stream.edge_stream_combine([(1.0, x), (0.5, a, s)], activation=activation,
                                                  gate=q if activation else None,
                                                  gate_rows=rows if activation else None)
            edge_stream.edge_stream_combine([(1.0, out), (-2.0, a)], out=acc)
        return (out, acc.clone())

    _check_replays(step, [x, a, s, q], seed=19)
