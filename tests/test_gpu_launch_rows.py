"""Launches that need more than one row of blocks give the same results.

HIP launches fewer than 2^32 work-items along each grid dimension, so a
kernel that takes one segment, row group or atom group per block runs on rows
of blocks along y once its work outgrows 16,777,215 blocks of 256 threads.
dpa4k_set_launch_row_limit lowers the blocks per row, so these tests reach
those grids at small sizes: every operator, on every launch path, must give
bit-identical results with 1 or 7 blocks per row and with the hardware limit.
(tests/test_gpu_large.py runs the same wrap at its real size.)
"""
from __future__ import annotations

import contextlib

import pytest
import torch

from bysj_amd import kernels, workloads
from bysj_amd.kernels import _C, _lib
from bysj_amd.kernels.gie import gie_zonal_scatter_rmsnorm
from parity import announce, assert_bitwise

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
LIMITS = (1, 7)


@contextlib.contextmanager
def row_limit(blocks: int):
    library = _lib.load()
    _lib.check(library.dpa4k_set_launch_row_limit(blocks))
    try:
        yield
    finally:
        _lib.check(library.dpa4k_set_launch_row_limit(0))


def _run_both(limit, compute):
    """compute() at the hardware limit and with `limit` blocks per row."""
    expected = compute()
    torch.cuda.synchronize()
    with row_limit(limit):
        actual = compute()
        torch.cuda.synchronize()
    return expected, actual


def _assert_all(expected, actual, what):
    assert len(expected) == len(actual)
    for i, (e, a) in enumerate(zip(expected, actual)):
        if e is None:
            assert a is None, f"{what}[{i}]"
            continue
        assert_bitwise(a, e, f"{what}[{i}]")


def _csr(n_nodes, mean, seed, hubs=0, hub_degree=0):
    degrees = workloads.poisson_degrees(n_nodes, mean, seed, minimum=0)
    if hubs:
        picks = workloads.rng(seed + 1).choice(n_nodes, size=hubs, replace=False)
        degrees[picks] = hub_degree
    offsets = torch.from_numpy(workloads.offsets_from_degrees(degrees))
    dst = torch.from_numpy(workloads.dst_from_degrees(degrees))
    return dst, offsets


def _leaf(tensor):
    return tensor.to(DEV).requires_grad_(True)


@pytest.mark.parametrize("limit", LIMITS)
@pytest.mark.parametrize("n_nodes,channels", [(700, 128), (5000, 128), (5000, 8), (1200, 640)])
@pytest.mark.parametrize("shuffle", [False, True])
def test_segment_sum_rows(limit, n_nodes, channels, shuffle):
    announce("rows segment_sum", limit, n_nodes, channels, shuffle)
    dst, offsets = _csr(n_nodes, 12, seed=n_nodes + channels)
    edges = dst.numel()
    gen = torch.Generator().manual_seed(7)
    src = torch.randn(edges, channels, generator=gen)
    edge_scale = torch.rand(edges, generator=gen) + 0.5
    node_scale = torch.rand(n_nodes, generator=gen) + 0.5
    grad = torch.randn(n_nodes, channels, generator=gen)
    order = None
    if shuffle:
        perm = torch.randperm(edges, generator=gen)
        order = perm.to(DEV)  # slot i holds edge perm[i]
        natural = torch.empty_like(dst)
        natural[perm] = dst
        dst = natural

    def compute():
        s, w, n = _leaf(src), _leaf(edge_scale), _leaf(node_scale)
        out = kernels.segment_sum(s, dst.to(DEV), offsets.to(DEV), w, n, order=order)
        out.backward(grad.to(DEV))
        return out.detach(), s.grad, w.grad, n.grad

    expected, actual = _run_both(limit, compute)
    _assert_all(expected, actual, "segment_sum")


@pytest.mark.parametrize("limit", LIMITS)
@pytest.mark.parametrize("channels", [8, 260])
@pytest.mark.parametrize("shuffle", [False, True])
def test_segment_softmax_rows(limit, channels, shuffle):
    announce("rows segment_softmax", limit, channels, shuffle)
    n_nodes = 13000 if channels == 8 else 1500  # more than three 4096-node plan tiles at C=8
    dst, offsets = _csr(n_nodes, 6, seed=channels, hubs=20, hub_degree=300)
    edges = dst.numel()
    gen = torch.Generator().manual_seed(11)
    logit = torch.randn(edges, channels, generator=gen) * 2
    env = torch.rand(edges, generator=gen) + 0.1
    env[::17] = 0.0
    null = torch.randn(n_nodes, channels, generator=gen)
    grad_alpha = torch.randn(edges, channels, generator=gen)
    grad_null = torch.randn(n_nodes, channels, generator=gen)
    order = None
    if shuffle:
        order = torch.randperm(edges, generator=gen).to(DEV)
    offsets_dev = offsets.to(DEV)

    def compute():
        lg, ev, nl = _leaf(logit), _leaf(env), _leaf(null)
        alpha, null_alpha = kernels.segment_softmax(lg, ev, offsets_dev, nl, order=order)
        torch.autograd.backward((alpha, null_alpha), (grad_alpha.to(DEV), grad_null.to(DEV)))
        # the unplanned launch path and the plan kernels themselves
        plain = _C.segment_softmax_forward(logit.to(DEV), env.to(DEV), offsets_dev, null.to(DEV), order)
        plan = _C.segment_softmax_plan(offsets_dev, edges, channels)
        words = plan.words[: 2 + plan.n_long].clone()
        return (alpha.detach(), null_alpha.detach(), lg.grad, ev.grad, nl.grad, plain[0], plain[1], words,
                torch.tensor([plan.n_long, plan.capacity]))

    expected, actual = _run_both(limit, compute)
    _assert_all(expected, actual, "segment_softmax")


@pytest.mark.parametrize("limit", LIMITS)
@pytest.mark.parametrize("primary", [True, False])
@pytest.mark.parametrize("shuffle", [False, True])
def test_gie_rows(limit, primary, shuffle):
    announce("rows gie", limit, primary, shuffle)
    n_nodes, channels = 900, 16
    dst, _ = _csr(n_nodes, 7, seed=3)
    edges = dst.numel()
    gen = torch.Generator().manual_seed(5)
    if primary:
        slots = torch.arange(1, 16, dtype=torch.int64)
        n_radial = 16
    else:
        slots = torch.tensor([0, 0, 0, 1, 1, 1, 1, 1, 2, 2, 2, 2, 2, 2, 2], dtype=torch.int64)
        n_radial = 3
    if shuffle:
        dst = dst[torch.randperm(edges, generator=gen)]
    zonal = torch.randn(edges, 15, generator=gen)
    radial = torch.randn(edges, n_radial, channels, generator=gen)
    inv = torch.rand(n_nodes, generator=gen) + 0.2
    scale = torch.rand(16 * channels, generator=gen) + 0.5
    grad = torch.randn(n_nodes, 16, channels, generator=gen)
    dst_dev, slots_dev = dst.to(DEV), slots.to(DEV)

    def compute():
        z, r, i = _leaf(zonal), _leaf(radial), _leaf(inv)
        out = kernels.gie_zonal_scatter(z, r, dst_dev, slots_dev, i)
        out.backward(grad.to(DEV))
        z2, r2, i2, s2 = _leaf(zonal), _leaf(radial), _leaf(inv), _leaf(scale)
        y = gie_zonal_scatter_rmsnorm(z2, r2, dst_dev, slots_dev, i2, s2)
        y.backward(grad.to(DEV))
        return out.detach(), z.grad, r.grad, i.grad, y.detach(), z2.grad, r2.grad, i2.grad, s2.grad

    expected, actual = _run_both(limit, compute)
    _assert_all(expected, actual, "gie")


@pytest.mark.parametrize("limit", LIMITS)
@pytest.mark.parametrize("width", [4, 64, 1024, 8200])
@pytest.mark.parametrize("use_scale", [True, False])
def test_rmsnorm_rows(limit, width, use_scale):
    announce("rows rmsnorm", limit, width, use_scale)
    rows = 3001
    gen = torch.Generator().manual_seed(width)
    x = torch.randn(rows, width, generator=gen)
    scale = torch.rand(width, generator=gen) + 0.5
    grad = torch.randn(rows, width, generator=gen)

    def compute():
        xv = _leaf(x)
        sv = _leaf(scale) if use_scale else None
        y = kernels.rmsnorm(xv, sv, 1e-6)
        y.backward(grad.to(DEV))
        return y.detach(), xv.grad, (sv.grad if use_scale else None)

    expected, actual = _run_both(limit, compute)
    _assert_all(expected, actual, "rmsnorm")


@pytest.mark.parametrize("limit", LIMITS)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_force_assembly_rows(limit, dtype):
    announce("rows force_assembly", limit, dtype)
    n_atoms = 3000
    dst, offsets = _csr(n_atoms, 20, seed=9)
    edges = dst.numel()
    gen = torch.Generator().manual_seed(13)
    src = torch.randint(0, n_atoms, (edges,), generator=gen)
    grad_edge = (torch.randn(edges, 3, generator=gen) * 0.5).to(dtype)
    edge_vec = torch.randn(edges, 3, generator=gen).to(dtype)
    args = [t.to(DEV) for t in (grad_edge, edge_vec, src, dst, offsets)]

    def compute():
        return kernels.force_assembly(*args)

    expected, actual = _run_both(limit, compute)
    _assert_all(expected, actual, "force_assembly")


@pytest.mark.parametrize("limit", LIMITS)
@pytest.mark.parametrize("channels", [64, 6])
def test_edge_stream_rows(limit, channels):
    from bysj_amd.kernels import edge_stream

    announce("rows edge stream", limit, channels)
    gen = torch.Generator(device=DEV)
    gen.manual_seed(31)
    shape = (3001, 9, channels)
    x, a = (torch.randn(*shape, generator=gen, device=DEV) for _ in range(2))
    s = torch.randn(shape[0], shape[1], 1, generator=gen, device=DEV)
    q = torch.randn(shape[0], 2, channels, generator=gen, device=DEV)
    rows = [-1, 0, 0, 0, 1, 1, 1, 1, 1]

    def compute():
        return (edge_stream.edge_stream_combine([(1.0, x), (0.5, a, s)]),
                edge_stream.edge_stream_combine([(1.0, x), (-1.0, a)], activation="gate", gate=q, gate_rows=rows))

    expected, actual = _run_both(limit, compute)
    _assert_all(expected, actual, "edge_stream")
