"""Parity at sizes past 32-bit offsets and past one row of blocks.

A 288 GB part holds operands far beyond 4 GiB, and the benchmark's roofline
shapes are that large (config 3R's radial input is 42.6 GB).  Each case here
generates its inputs on the device at such a size, runs the operator and its
gradient through kernels.*, and checks sampled segments, rows or atoms --
the first and last ones, the ones around a boundary of the case and random
ones -- against the CPU oracle run on the sub-graph those samples span
(each sampled output depends only on the edges of its own segment, so the
sub-graph gives the oracle the same terms).  A segment longer than 2 GiB is
checked whole on the device against an fp64 restatement of the closed form.

What each case crosses:
  segment_softmax  logits of 4.8 GB (> 2^32 bytes) with one 2.1 GB segment
                   (> 2^31 bytes): the buffer windows of the streaming path
  segment_sum      src of 2.4e9 floats (> 2^31 elements) through a random order
  rmsnorm          67.1M rows: the forward needs two rows of blocks
  gie              67.1M nodes (two rows of blocks, both backward kernels),
                   and config 3R's 42.6 GB radial input through a shuffled dst
  force_assembly   190M edges: grad_edge and edge_vec past 2^31 bytes (fp32)
                   and 2^32 bytes (fp64)
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from bysj_amd import kernels, workloads
from oracle import gie as gie_ref
from oracle import loops
from oracle import segment as ref
from oracle.rmsnorm import rmsnorm as rmsnorm_ref
from oracle.rmsnorm import rmsnorm_backward_reference
from parity import FP32_RTOL, FP32_SCALE, announce, assert_bitwise, assert_close_scaled

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
ROW_256 = 4294967295 // 256  # blocks of 256 threads in one grid row
ROW_64 = 4294967295 // 64


@pytest.fixture(autouse=True)
def _release():
    yield
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def _generator(seed: int) -> torch.Generator:
    gen = torch.Generator(device=DEV)
    gen.manual_seed(seed)
    return gen


def _samples(n: int, seed: int, around=(), count: int = 24, exclude=()) -> torch.Tensor:
    picks = {0, 1, 2, n - 3, n - 2, n - 1}
    for center in around:
        picks.update(range(center - 3, center + 4))
    picks.update(workloads.rng(seed).integers(0, n, size=count).tolist())
    picks = sorted(p for p in picks if 0 <= p < n and p not in set(exclude))
    return torch.tensor(picks, dtype=torch.int64)


def _sub_csr(offsets: torch.Tensor, nodes: torch.Tensor):
    """Slots of `nodes` in CSR order, and the sub-graph's offsets and dst."""
    begins, ends = offsets[nodes], offsets[nodes + 1]
    degrees = ends - begins
    slots = torch.cat([torch.arange(b, e, dtype=torch.int64) for b, e in zip(begins.tolist(), ends.tolist())])
    sub_offsets = torch.cat([torch.zeros(1, dtype=torch.int64), degrees.cumsum(0)])
    sub_dst = torch.repeat_interleave(torch.arange(nodes.numel(), dtype=torch.int64), degrees)
    return slots, sub_offsets, sub_dst


def _take(tensor: torch.Tensor, index: torch.Tensor) -> torch.Tensor:
    return tensor.detach()[index.to(tensor.device)].cpu()


def _close_on_device(actual: torch.Tensor, expected: torch.Tensor, what: str) -> None:
    """The fp32 rule, evaluated on the device for operands too large to copy."""
    expected = expected.double()
    budget = FP32_RTOL * expected.abs() + FP32_SCALE * expected.abs().max()
    error = (actual.detach().double() - expected).abs()
    bad = int((error > budget).sum())
    assert bad == 0, f"{what}: {bad} of {expected.numel()} elements outside the fp32 rule"


def test_segment_softmax_past_32bit_offsets():
    channels = 8
    hub_rows = (1 << 31) // (4 * channels) + 4099  # one segment with more than 2 GiB of logits
    degrees = workloads.poisson_degrees(1_300_000, 64, seed=31, minimum=0)
    hub = degrees.shape[0] // 2
    degrees = np.insert(degrees, hub, hub_rows)
    n_nodes = degrees.shape[0]
    offsets = torch.from_numpy(workloads.offsets_from_degrees(degrees))
    edges = int(offsets[-1])
    assert edges * channels * 4 > (1 << 32) + (1 << 28)
    announce("large segment_softmax", edges, n_nodes, hub_rows)
    gen = _generator(31)
    logit = torch.randn(edges, channels, device=DEV, generator=gen).mul_(2.0).requires_grad_()
    env = torch.rand(edges, device=DEV, generator=gen).add_(0.1).requires_grad_()
    null = torch.randn(n_nodes, channels, device=DEV, generator=gen).requires_grad_()
    alpha, null_alpha = kernels.segment_softmax(logit, env, offsets.to(DEV), null)
    grad_alpha = torch.randn(edges, channels, device=DEV, generator=gen)
    grad_null = torch.randn(n_nodes, channels, device=DEV, generator=gen)
    torch.autograd.backward((alpha, null_alpha), (grad_alpha, grad_null))
    torch.cuda.synchronize()

    nodes = _samples(n_nodes, 31, around=(hub,), exclude=(hub,))
    slots, sub_offsets, sub_dst = _sub_csr(offsets, nodes)
    lg, ev, nl = _take(logit, slots), _take(env, slots), _take(null, nodes)
    e_alpha, e_null = ref.segment_softmax_reference(lg, ev, sub_dst, sub_offsets, nl)
    assert_close_scaled(_take(alpha, slots), e_alpha, what="sampled alpha")
    assert_close_scaled(_take(null_alpha, nodes), e_null, what="sampled null_alpha")
    g_logit, g_env, g_null = ref.segment_softmax_backward_reference(
        _take(grad_alpha, slots), lg, ev, sub_dst, sub_offsets, nl, _take(grad_null, nodes))
    assert_close_scaled(_take(logit.grad, slots), g_logit, what="sampled grad_logit")
    assert_close_scaled(_take(env.grad, slots), g_env, what="sampled grad_env")
    assert_close_scaled(_take(null.grad, nodes), g_null, what="sampled grad_null")

    # the hub, whole, against the closed form in fp64 on the device
    b, e = int(offsets[hub]), int(offsets[hub + 1])
    with torch.no_grad():
        weight = logit[b:e].double() + 2.0 * env[b:e].double().log().unsqueeze(1)
        n0 = null[hub].double()
        peak = torch.maximum(weight.max(0).values, n0)
        weight.sub_(peak).exp_()
        total = weight.sum(0) + (n0 - peak).exp()
        weight.div_(total)  # alpha in fp64
        a0 = (n0 - peak).exp() / total
        _close_on_device(alpha[b:e], weight, "hub alpha")
        _close_on_device(null_alpha[hub], a0, "hub null_alpha")
        g = grad_alpha[b:e].double()
        g0 = grad_null[hub].double()
        s = (weight * g).sum(0) + a0 * g0
        g.sub_(s).mul_(weight)  # d logit
        _close_on_device(logit.grad[b:e], g, "hub grad_logit")
        _close_on_device(env.grad[b:e], 2.0 / env[b:e].double() * g.sum(1), "hub grad_env")
        _close_on_device(null.grad[hub], a0 * (g0 - s), "hub grad_null")


def test_segment_sum_past_2_31_elements():
    channels = 128
    degrees = workloads.poisson_degrees(110_000, 170, seed=41, minimum=0)
    n_nodes = degrees.shape[0]
    offsets = torch.from_numpy(workloads.offsets_from_degrees(degrees))
    edges = int(offsets[-1])
    assert edges * channels > (1 << 31) + (1 << 27)
    announce("large segment_sum", edges, n_nodes, channels)
    gen = _generator(41)
    src = torch.randn(edges, channels, device=DEV, generator=gen).requires_grad_()
    edge_scale = torch.rand(edges, device=DEV, generator=gen).add_(0.5).requires_grad_()
    node_scale = torch.rand(n_nodes, device=DEV, generator=gen).add_(0.5).requires_grad_()
    order = torch.randperm(edges, device=DEV, generator=gen)  # slot i holds edge order[i]
    dst = torch.empty(edges, dtype=torch.int64, device=DEV)
    dst[order] = torch.repeat_interleave(torch.arange(n_nodes, device=DEV), torch.from_numpy(degrees).to(DEV))
    out = kernels.segment_sum(src, dst, offsets.to(DEV), edge_scale, node_scale, order=order)
    grad = torch.randn(n_nodes, channels, device=DEV, generator=gen)
    out.backward(grad)
    torch.cuda.synchronize()

    nodes = _samples(n_nodes, 41, count=40)
    slots, sub_offsets, sub_dst = _sub_csr(offsets, nodes)
    picked = _take(order, slots)
    assert int(picked.max()) * channels >= 1 << 31, "the samples must reach past 2^31 elements"
    s_src, s_w, s_n = _take(src, picked), _take(edge_scale, picked), _take(node_scale, nodes)
    expected = ref.segment_sum_reference(s_src, sub_dst, sub_offsets, s_w, s_n)
    assert_bitwise(_take(out, nodes), expected, "sampled forward (sequential fp32 chain)")
    g_src, g_w, g_n = ref.segment_sum_backward_reference(_take(grad, nodes), s_src, sub_dst, sub_offsets, s_w, s_n)
    assert_close_scaled(_take(src.grad, picked), g_src, what="sampled grad_src")
    assert_close_scaled(_take(edge_scale.grad, picked), g_w, what="sampled grad_edge_scale")
    assert_close_scaled(_take(node_scale.grad, nodes), g_n, what="sampled grad_node_scale")


def test_rmsnorm_two_rows_of_blocks():
    width = 4
    rows = ROW_256 * 4 + 4099  # four rows per block: more blocks than one grid row holds
    announce("large rmsnorm", rows, width)
    gen = _generator(51)
    x = torch.randn(rows, width, device=DEV, generator=gen).requires_grad_()
    scale = torch.rand(width, device=DEV, generator=gen).add_(0.5)
    y = kernels.rmsnorm(x, scale, 1e-6)
    grad = torch.randn(rows, width, device=DEV, generator=gen)
    y.backward(grad)
    torch.cuda.synchronize()

    # two grid rows of equal length: the second starts at row rows // 2 (rounded up to a block)
    picks = _samples(rows, 51, around=(rows // 2, rows - 4099), count=256)
    xs = _take(x, picks)
    assert_close_scaled(_take(y, picks), rmsnorm_ref(xs, scale.cpu(), 1e-6), what="sampled rows")
    grad_x, _ = rmsnorm_backward_reference(_take(grad, picks), xs, scale.cpu(), 1e-6)
    assert_close_scaled(_take(x.grad, picks), grad_x, what="sampled grad_x")


def _gie_case(n_nodes, mean, n_radial, slots, channels, seed, shuffle, around):
    degrees = workloads.poisson_degrees(n_nodes, mean, seed=seed, minimum=0)
    offsets = torch.from_numpy(workloads.offsets_from_degrees(degrees))
    edges = int(offsets[-1])
    n_rows = slots.numel()
    announce("large gie", n_nodes, edges, n_radial, channels, shuffle)
    gen = _generator(seed)
    zonal = torch.randn(edges, n_rows, device=DEV, generator=gen).requires_grad_()
    radial = torch.randn(edges, n_radial, channels, device=DEV, generator=gen).requires_grad_()
    inv = torch.rand(n_nodes, device=DEV, generator=gen).add_(0.2).requires_grad_()
    sorted_dst = torch.repeat_interleave(torch.arange(n_nodes, device=DEV), torch.from_numpy(degrees).to(DEV))
    if shuffle:
        perm = torch.randperm(edges, device=DEV, generator=gen)  # edge perm[i] sits in slot i
        dst = torch.empty_like(sorted_dst)
        dst[perm] = sorted_dst
    else:
        perm, dst = None, sorted_dst
    del sorted_dst
    out = kernels.gie_zonal_scatter(zonal, radial, dst, slots.to(DEV), inv)
    grad = torch.randn(n_nodes, n_rows + 1, channels, device=DEV, generator=gen)
    out.backward(grad)
    torch.cuda.synchronize()

    nodes = _samples(n_nodes, seed, around=around)
    slot_ids, _, sub_dst = _sub_csr(offsets, nodes)
    picked = slot_ids if perm is None else _take(perm, slot_ids)
    s_zonal, s_radial, s_inv = _take(zonal, picked), _take(radial, picked), _take(inv, nodes)
    expected = gie_ref.zonal_scatter_reference(s_zonal, s_radial, sub_dst, slots, s_inv)
    assert_close_scaled(_take(out, nodes), expected, what="sampled output")
    g_zonal, g_radial, g_inv = gie_ref.zonal_scatter_backward_reference(
        _take(grad, nodes), s_zonal, s_radial, sub_dst, slots, s_inv)
    assert_close_scaled(_take(zonal.grad, picked), g_zonal, what="sampled grad_zonal")
    assert_close_scaled(_take(radial.grad, picked), g_radial, what="sampled grad_radial")
    assert_close_scaled(_take(inv.grad, nodes), g_inv, what="sampled grad_inv")
    return picked


@pytest.mark.parametrize("shared", [False, True])
def test_gie_two_rows_of_blocks(shared):
    # four nodes per 256-thread block (forward, distinct-slot backward) and one
    # node per 64-thread block (shared-slot backward): both need two grid rows
    n_nodes = ROW_256 * 4 + 1001
    assert n_nodes > ROW_64
    slots = torch.tensor([0, 0] if shared else [0, 1], dtype=torch.int64)
    # both kernels' second grid row starts within three nodes of n_nodes // 2
    _gie_case(n_nodes, 1.0, 1 if shared else 2, slots, 4, seed=61 + shared, shuffle=False,
              around=(n_nodes // 2,))


def test_gie_config3R_radial_past_32bit_offsets():
    # config 3R's primary shape: 114,688 nodes of ~90 edges, radial [E, 16, 64] (42.6 GB)
    slots = torch.arange(1, 16, dtype=torch.int64)
    picked = _gie_case(114_688, 90.5, 16, slots, 64, seed=71, shuffle=True, around=())
    assert int(picked.max()) * 16 * 64 * 4 >= 1 << 32, "the samples must reach past 2^32 bytes"


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_force_assembly_past_32bit_offsets(dtype):
    n_atoms, edges = 9_500_000, 190_000_000
    announce("large force_assembly", n_atoms, edges, dtype)
    degrees = workloads.poisson_degrees(n_atoms, edges / n_atoms, seed=81, minimum=0)
    dst_offsets = torch.from_numpy(workloads.offsets_from_degrees(degrees))
    edges = int(dst_offsets[-1])
    assert edges * 3 * 4 > (1 << 31)
    gen = _generator(81)
    dst = torch.repeat_interleave(torch.arange(n_atoms, device=DEV), torch.from_numpy(degrees).to(DEV))
    src = torch.randint(0, n_atoms, (edges,), device=DEV, generator=gen)
    grad_edge = torch.randn(edges, 3, device=DEV, generator=gen, dtype=dtype).mul_(0.5)
    edge_vec = torch.randn(edges, 3, device=DEV, generator=gen, dtype=dtype)
    src_order, src_offsets = kernels.group_by_source(src, n_atoms)
    force, virial = kernels.force_assembly(grad_edge, edge_vec, src, dst, dst_offsets.to(DEV), src_offsets,
                                           src_order)
    torch.cuda.synchronize()

    atoms = _samples(n_atoms, 81, count=32)
    s_offsets = src_offsets.cpu()
    dst_side = [torch.arange(int(dst_offsets[a]), int(dst_offsets[a + 1])) for a in atoms.tolist()]
    src_side = [_take(src_order, torch.arange(int(s_offsets[a]), int(s_offsets[a + 1]))) for a in atoms.tolist()]
    picked = torch.unique(torch.cat(dst_side + src_side))
    assert int(picked.max()) * 3 * grad_edge.element_size() >= 1 << 31
    # relabel: sampled atom i -> i, every other atom -> len(atoms) (collects terms not checked)
    label = {a: i for i, a in enumerate(atoms.tolist())}
    other = atoms.numel()

    def relabel(ids):
        return torch.tensor([label.get(v, other) for v in ids.tolist()], dtype=torch.int64)

    e_force, e_virial = loops.force_assembly_loop(
        _take(grad_edge, picked), _take(edge_vec, picked), relabel(_take(src, picked)),
        relabel(_take(dst, picked)), other + 1)
    rule = {} if dtype == torch.float32 else {"rtol": 1e-12, "scale": 1e-12}
    assert_close_scaled(_take(force, atoms), e_force[:other], what="sampled force", **rule)
    assert_close_scaled(_take(virial, atoms), e_virial[:other], what="sampled virial", **rule)
