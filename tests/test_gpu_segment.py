"""GPU parity of the CSR helpers, segment_sum, segment_softmax and force_assembly.

Every case compares the gfx950 path (through kernels.* -> kernels._C ->
libdpa4k.so) with the CPU oracle on the same seeded inputs: bit for bit for
indices and for the sequential segment_sum forward, the fp32 rule against the
oracle and an fp64 ground truth otherwise.  Shapes follow the reference's
device tests (tests/csrc/accuracy/test_segment_ops_accuracy.py).
"""
from __future__ import annotations

import importlib

import numpy as np
import pytest
import torch

from bysj_amd import kernels, workloads
from oracle import gie as gie_ref
from oracle import loops
from oracle import segment as ref
from closed_forms import segment_softmax_backward_f64, segment_sum_backward_f64
from parity import announce, assert_bitwise, assert_close_scaled, assert_fp64, assert_gradient

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
segment_mod = importlib.import_module("bysj_amd.kernels.segment")


def _graph(sizes):
    sizes = torch.tensor(sizes, dtype=torch.int64)
    dst = torch.repeat_interleave(torch.arange(sizes.numel(), dtype=torch.int64), sizes)
    return dst, torch.cat([torch.zeros(1, dtype=torch.int64), sizes.cumsum(0)])


def _shuffled(dst_sorted: torch.Tensor, seed: int):
    """Natural order = a seeded permutation of a grouped list; CSR via stable argsort."""
    gen = torch.Generator().manual_seed(seed)
    perm = torch.randperm(dst_sorted.numel(), generator=gen)
    dst = dst_sorted[perm]
    n = int(dst_sorted.max()) + 1 if dst_sorted.numel() else 1
    order, offsets = ref.group_by_source(dst, n)
    return dst, order, offsets


# ---------------------------------------------------------------------------
# CSR construction (bit-exact)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("edges,nodes,seed", [(0, 5, 0), (1, 1, 1), (1000, 37, 2), (200000, 5000, 3),
                                              (300000, 300001, 4)])
def test_segment_offsets_and_grouping_bit_exact(edges, nodes, seed):
    announce("csr", edges, nodes, seed)
    gen = torch.Generator().manual_seed(seed)
    keys = torch.randint(0, nodes, (edges,), generator=gen, dtype=torch.int64)
    offsets = kernels.segment_offsets(keys.to(DEV), nodes)
    assert_bitwise(offsets, ref.segment_offsets(keys, nodes), "segment_offsets")
    order, src_offsets = kernels.group_by_source(keys.to(DEV), nodes)
    e_order, e_offsets = ref.group_by_source(keys, nodes)
    assert_bitwise(order, e_order, "group_by_source order")
    assert_bitwise(src_offsets, e_offsets, "group_by_source offsets")


def _check_grouping_against_numpy(keys: np.ndarray, nodes: int, what: str) -> None:
    """group_by_source and segment_offsets of int64 `keys` against numpy's stable argsort and bincount."""
    device_keys = torch.from_numpy(keys).to(DEV)
    expected_offsets = np.concatenate([[0], np.cumsum(np.bincount(keys, minlength=nodes))]).astype(np.int64)
    expected_order = np.argsort(keys, kind="stable").astype(np.int64)
    assert_bitwise(kernels.segment_offsets(device_keys, nodes), torch.from_numpy(expected_offsets),
                   f"{what}: segment_offsets")
    order, offsets = kernels.group_by_source(device_keys, nodes)
    assert_bitwise(offsets, torch.from_numpy(expected_offsets), f"{what}: group_by_source offsets")
    assert_bitwise(order, torch.from_numpy(expected_order), f"{what}: group_by_source order")
    again, _ = kernels.group_by_source(device_keys, nodes)
    assert_bitwise(again, order, f"{what}: run to run")


@pytest.mark.parametrize("edges,nodes", [
    (8191, 2), (8192, 513), (8193, 65536), (100000, 1), (250000, 65537), (600000, 2**20),
    (2_200_000, 2**21),        # (E - 1) << fine_bits passes 32 bits: 64-bit packed entries
    (300000, 2**21 + 5),       # past 21 key bits: least-significant-digit passes
    (150000, 2**26), (40000, 2**27 + 3),
])
def test_counting_sort_paths_bit_exact(edges, nodes):
    """Every path of the device counting sort (two-level with 32- and 64-bit packed entries, the LSD
    passes, partial tiles, one node) against numpy's stable argsort, on unsorted and sorted keys."""
    announce("counting sort", edges, nodes)
    keys = workloads.rng(edges % 1000 + nodes % 1000).integers(0, nodes, size=edges).astype(np.int64)
    _check_grouping_against_numpy(keys, nodes, f"random E={edges} N={nodes}")
    _check_grouping_against_numpy(np.sort(keys), nodes, f"sorted E={edges} N={nodes}")


def test_counting_sort_skewed_and_sparse_keys():
    """Hubs that fill a bucket many times over (the bucket-local pass runs chunk after chunk), a single
    key everywhere, and sparse keys over millions of nodes (long runs of empty segments, sorted and not,
    filled cooperatively instead of by one thread)."""
    announce("counting sort: skewed and sparse")
    gen = workloads.rng(77)
    hubs = np.concatenate([np.full(300000, 4097), np.full(100000, 5), gen.integers(0, 65536, 200000)])
    gen.shuffle(hubs)
    _check_grouping_against_numpy(hubs.astype(np.int64), 65536, "hubs")
    _check_grouping_against_numpy(np.full(70000, 3, dtype=np.int64), 4, "one key")
    sparse = gen.integers(0, 30_000_000, 50).astype(np.int64)
    _check_grouping_against_numpy(sparse, 30_000_000, "sparse unsorted")
    _check_grouping_against_numpy(np.sort(sparse), 30_000_000, "sparse sorted")
    _check_grouping_against_numpy(np.array([0, 9_999_999], dtype=np.int64), 10_000_000, "two keys, ends")


@pytest.mark.parametrize("edges,nodes", [(700_000, 128), (800_000, 128), (6_300_000, 2**16), (8_388_608, 2**16),
                                         (9_000_000, 4096), (3_000_000, 2**17), (12_000_000, 2**17)])
def test_counting_sort_bucket_chunks(edges, nodes):
    """Buckets that average just under and just over 95% of the gather's 6144-element chunk (the two
    chunk sizes of the grouped path), and config-4-sized buckets past it, with one bucket pushed over
    the chunk so that it takes the multi-chunk path beside ones that do not; then the gather's wider
    instances: 1,024 tiles exactly, more than 1,024 tiles, 7-bit fine digits, and both at once with
    every bucket longer than a chunk (a config-4R-sized list)."""
    announce("counting sort: bucket chunks", edges, nodes)
    keys = workloads.rng(edges % 997 + nodes).integers(0, nodes, size=edges).astype(np.int64)
    keys[: edges // 64] = 5
    _check_grouping_against_numpy(keys, nodes, f"chunks E={edges} N={nodes}")


@pytest.mark.parametrize("edges,nodes", [(16_777_217, 2**16), (2_000_000, 2**18)])
def test_counting_sort_past_the_grouped_limits(edges, nodes):
    """Keys that the grouped path does not take: more tiles than it holds (2,048 tiles of 8,192 keys;
    one key past the limit) and 8 fine bits.  The four-launch build."""
    announce("counting sort: past the grouped limits", edges, nodes)
    keys = workloads.rng(edges % 991 + nodes).integers(0, nodes, size=edges).astype(np.int64)
    _check_grouping_against_numpy(keys, nodes, f"four-launch E={edges} N={nodes}")


def test_group_by_key_async_status_and_capture():
    """The asynchronous build reports the status bits on the device, allocates nothing when given its
    buffers, and replays from a HIP graph with the same result as the synchronous call."""
    from bysj_amd.kernels import _C, _lib

    announce("group_by_key async")
    keys = torch.from_numpy(workloads.rng(5).integers(0, 70000, size=90000).astype(np.int64)).to(DEV)
    order, offsets = kernels.group_by_source(keys, 70000)
    buffers = dict(order=torch.empty_like(order), offsets=torch.empty_like(offsets),
                   status=torch.full((1,), 99, dtype=torch.int32, device=DEV),
                   workspace=torch.empty(_lib.load().dpa4k_group_by_key_workspace_size(90000, 70000),
                                         dtype=torch.uint8, device=DEV))
    _C.group_by_key_async(keys, 70000, **buffers)
    assert int(buffers["status"].item()) == 2  # unsorted, in range
    assert_bitwise(buffers["order"], order, "async order")
    assert_bitwise(buffers["offsets"], offsets, "async offsets")
    graph = torch.cuda.CUDAGraph()
    fresh = {k: (torch.zeros_like(v) if k != "workspace" else v) for k, v in buffers.items()}
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        _C.group_by_key_async(keys, 70000, **fresh)
    for replay in range(3):
        fresh["order"].zero_()
        fresh["status"].fill_(99)
        graph.replay()
        torch.cuda.synchronize()
        assert_bitwise(fresh["order"], order, f"replay {replay} order")
        assert_bitwise(fresh["offsets"], offsets, f"replay {replay} offsets")
        assert int(fresh["status"].item()) == 2
    sorted_keys = torch.sort(keys).values
    _C.group_by_key_async(sorted_keys, 70000, **buffers)
    assert int(buffers["status"].item()) == 0
    bad = keys.clone()
    bad[1234] = 70000
    _C.group_by_key_async(bad, 70000, **buffers)
    assert int(buffers["status"].item()) & 1 == 1
    bad[1234] = -3
    _C.group_by_key_async(bad, 70000, **buffers)
    assert int(buffers["status"].item()) & 1 == 1


@pytest.mark.parametrize("sort", [False, True])
def test_destination_grouping(sort):
    """Offsets equal segment_offsets; the order is None exactly when dst is non-decreasing."""
    announce("destination grouping", sort)
    gen = torch.Generator().manual_seed(21)
    keys = torch.randint(0, 700, (50000,), generator=gen, dtype=torch.int64)
    if sort:
        keys = torch.sort(keys).values
    offsets, order = segment_mod.destination_grouping(keys.to(DEV), 700)
    e_order, e_offsets = ref.group_by_source(keys, 700)
    assert_bitwise(offsets, e_offsets, "offsets")
    if sort:
        assert order is None
    else:
        assert_bitwise(order, e_order, "order")
    with pytest.raises(ValueError, match="node range"):
        segment_mod.destination_grouping(torch.tensor([0, 700], device=DEV), 700)


def test_grouping_known_answer_and_range_errors():
    announce("csr known answer")
    src = torch.tensor([2, 0, 2, 1, 0], dtype=torch.int64, device=DEV)
    order, offsets = kernels.group_by_source(src, 3)
    assert offsets.cpu().tolist() == [0, 2, 3, 5]
    assert order.cpu().tolist() == [1, 4, 3, 0, 2]
    dst, expected = _graph([2, 0, 3])
    assert kernels.segment_offsets(dst.to(DEV), 3).cpu().tolist() == expected.tolist()
    with pytest.raises(ValueError):
        kernels.segment_offsets(torch.tensor([0, 3], dtype=torch.int64, device=DEV), 3)
    with pytest.raises(ValueError):
        kernels.group_by_source(torch.tensor([-1, 0], dtype=torch.int64, device=DEV), 3)


# ---------------------------------------------------------------------------
# segment_sum
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("channels", [1, 3, 8, 64, 128, 640, 1024, 2052, 4100])
@pytest.mark.parametrize("scales", [False, True])
def test_segment_sum_forward_bit_exact(channels, scales):
    announce("segment_sum fwd", channels, scales)
    case = workloads.segment_sum_config(n_nodes=97, channels=channels, seed=channels, scales=scales)
    d = {k: (v.to(DEV) if v is not None else None) for k, v in case.items()}
    out = kernels.segment_sum(d["src"], d["dst"], d["offsets"], d["edge_scale"], d["node_scale"])
    expected = ref.segment_sum_reference(case["src"], case["dst"], case["offsets"], case["edge_scale"],
                                         case["node_scale"])
    assert_bitwise(out, expected, "segment_sum vs sequential oracle")


def test_segment_sum_reference_cases_and_empty_segments():
    announce("segment_sum reference cases")
    for channels in (1, 3, 64, 640):
        dst, offsets = _graph([2, 0, 3])
        gen = torch.Generator().manual_seed(channels)
        src = torch.randn(5, channels, generator=gen)
        edge_scale = torch.rand(5, generator=gen) + 0.5
        node_scale = torch.rand(3, generator=gen) + 0.5
        out = kernels.segment_sum(src.to(DEV), dst.to(DEV), offsets.to(DEV), edge_scale.to(DEV), node_scale.to(DEV))
        assert_bitwise(out, ref.segment_sum_reference(src, dst, offsets, edge_scale, node_scale), "reference case")
        assert out[1].count_nonzero().item() == 0
    # no edges at all: zeros (times the node scale)
    src = torch.empty(0, 4)
    dst = torch.empty(0, dtype=torch.int64)
    offsets = torch.zeros(4, dtype=torch.int64)
    out = kernels.segment_sum(src.to(DEV), dst.to(DEV), offsets.to(DEV))
    assert out.shape == (3, 4) and out.count_nonzero().item() == 0


@pytest.mark.parametrize("channels", [5, 128])
def test_segment_sum_with_order_is_bit_exact(channels):
    announce("segment_sum order", channels)
    degrees = workloads.poisson_degrees(211, 12.0, seed=5)
    dst_sorted = torch.from_numpy(workloads.dst_from_degrees(degrees))
    dst, order, offsets = _shuffled(dst_sorted, seed=7)
    gen = torch.Generator().manual_seed(9)
    src = torch.randn(dst.numel(), channels, generator=gen)
    w = torch.rand(dst.numel(), generator=gen) + 0.5
    s = torch.rand(211, generator=gen) + 0.5
    out = kernels.segment_sum(src.to(DEV), dst.to(DEV), offsets.to(DEV), w.to(DEV), s.to(DEV), order=order.to(DEV))
    assert_bitwise(out, ref.segment_sum_reference(src, dst, offsets, w, s), "segment_sum with order")


@pytest.mark.parametrize("channels", [64, 128, 256])
def test_segment_sum_nan_edge_scale_propagates_with_order(channels):
    """A NaN in edge_scale reaches the output of its segment, with or without an order, on the
    small-grid staged path (fewer than 4096 segments, 64-256 channels) as in the oracle's
    index_add_ chain: the staged kernel's skip flag for bad order entries is not a NaN weight."""
    announce("segment_sum NaN edge_scale", channels)
    degrees = workloads.poisson_degrees(211, 12.0, seed=channels)
    dst_sorted = torch.from_numpy(workloads.dst_from_degrees(degrees))
    dst, order, offsets = _shuffled(dst_sorted, seed=channels)
    gen = torch.Generator().manual_seed(channels)
    src = torch.randn(dst.numel(), channels, generator=gen)
    w = torch.rand(dst.numel(), generator=gen) + 0.5
    w[[3, 500, dst.numel() - 1]] = float("nan")
    s = torch.rand(211, generator=gen) + 0.5
    expected = ref.segment_sum_reference(src, dst, offsets, w, s)
    assert bool(torch.isnan(expected).any())
    with_order = kernels.segment_sum(src.to(DEV), dst.to(DEV), offsets.to(DEV), w.to(DEV), s.to(DEV),
                                     order=order.to(DEV))
    assert_bitwise(with_order, expected, "NaN edge_scale with order vs oracle")
    # the same edges in their grouped (natural) order, without an order argument
    grouped = order.to(DEV)
    natural = kernels.segment_sum(src.to(DEV)[grouped].contiguous(), dst_sorted.to(DEV), offsets.to(DEV),
                                  w.to(DEV)[grouped].contiguous(), s.to(DEV))
    assert_bitwise(natural, with_order, "order=None on the grouped copy")


def test_segment_sum_large_graph_against_fp64_truth():
    announce("segment_sum fp64 truth")
    gen = torch.Generator().manual_seed(11)
    atoms, edges, channels = 64, 4096, 32
    dst = torch.sort(torch.randint(0, atoms, (edges,), generator=gen)).values
    offsets = ref.segment_offsets(dst, atoms)
    src = torch.randn(edges, channels, generator=gen)
    node_scale = torch.rand(atoms, generator=gen) + 0.5
    out = kernels.segment_sum(src.to(DEV), dst.to(DEV), offsets.to(DEV), None, node_scale.to(DEV))
    truth = loops.segment_sum_loop(src, dst, atoms, None, node_scale)
    assert_close_scaled(out, truth, what="vs fp64 truth")


def test_segment_sum_config1_full_size_and_determinism():
    announce("segment_sum config 1")
    case = workloads.segment_sum_config(seed=0)
    d = {k: (v.to(DEV) if v is not None else None) for k, v in case.items()}
    first = kernels.segment_sum(d["src"], d["dst"], d["offsets"])
    second = kernels.segment_sum(d["src"], d["dst"], d["offsets"])
    assert_bitwise(first, second, "run-to-run")
    assert_bitwise(first, ref.segment_sum_reference(case["src"], case["dst"], case["offsets"]), "config 1")


@pytest.mark.parametrize("channels", [64, 128, 256])
@pytest.mark.parametrize("use_order", [False, True])
def test_segment_sum_workgroup_path_long_segments(channels, use_order):
    """Small grids take the workgroup-per-segment kernels; segments longer than one LDS batch
    repeat the forward's staging step.  The same graph padded past the small-grid limit with empty
    segments takes the lane-group forward (the backward keeps its workgroup kernel), and the
    results must agree bit for bit (forward, grad_src)."""
    announce("segment_sum workgroup path", channels, use_order)
    gen = torch.Generator().manual_seed(channels + int(use_order))
    degrees = np.array([0, 1, 2, 300, 1000, 45, 0, 129, 64, 33, 7, 511], dtype=np.int64)
    nodes = degrees.size
    dst_sorted = torch.from_numpy(workloads.dst_from_degrees(degrees))
    if use_order:
        dst, order, offsets = _shuffled(dst_sorted, seed=channels)
    else:
        dst, order, offsets = dst_sorted, None, ref.segment_offsets(dst_sorted, nodes)
    edges = dst.numel()
    src = torch.randn(edges, channels, generator=gen)
    w = torch.rand(edges, generator=gen) + 0.5
    s = torch.rand(nodes, generator=gen) + 0.5
    g = torch.randn(nodes, channels, generator=gen)
    o = None if order is None else order.to(DEV)
    x = src.to(DEV).requires_grad_(True)
    wd = w.to(DEV).requires_grad_(True)
    sd = s.to(DEV).requires_grad_(True)
    out = kernels.segment_sum(x, dst.to(DEV), offsets.to(DEV), wd, sd, order=o)
    assert_bitwise(out, ref.segment_sum_reference(src, dst, offsets, w, s), "workgroup-path forward")
    grads = torch.autograd.grad(out, (x, wd, sd), g.to(DEV))
    e_src, e_w, e_s = ref.segment_sum_backward_reference(g, src, dst, offsets, w, s)
    assert_bitwise(grads[0], e_src, "workgroup-path grad_src")
    assert_close_scaled(grads[1], e_w, what="workgroup-path grad_edge_scale")
    assert_close_scaled(grads[2], e_s, what="workgroup-path grad_node_scale")
    # the same edges under 5000 more (empty) segments: the lane-group kernels
    pad = 5000
    offsets_big = torch.cat([offsets, offsets[-1:].expand(pad)])
    s_big = torch.cat([s, torch.ones(pad)])
    g_big = torch.cat([g, torch.zeros(pad, channels)])
    native = kernels._C
    big = native.segment_sum_forward(src.to(DEV), offsets_big.to(DEV), w.to(DEV), s_big.to(DEV), o)
    assert_bitwise(big[:nodes], out, "lane-group vs workgroup forward")
    grads_big = native.segment_sum_backward(g_big.to(DEV), src.to(DEV), dst.to(DEV), offsets_big.to(DEV), w.to(DEV),
                                            s_big.to(DEV), True, o, want_edge_scale_grad=True)
    assert_bitwise(grads_big[0], grads[0], "padded grid vs small grid grad_src")
    assert_close_scaled(grads_big[2], grads[1], what="padded grid vs small grid grad_edge_scale")
    assert_close_scaled(grads_big[1][:nodes], grads[2], what="padded grid vs small grid grad_node_scale")


@pytest.mark.parametrize("channels", [3, 5, 8, 32, 64, 128])
@pytest.mark.parametrize("scales", [False, True])
def test_segment_sum_large_grid_natural_order_rounds(channels, scales):
    """Grids past the small-grid limit (N * lanes per segment / 64 >= 2048 waves) read rows in natural
    order 32 slots a round: segments shorter than a round, of exactly one, and of several rounds plus a
    tail, at widths of one float per lane (C = 3, 5) to one float4 per lane (C = 128)."""
    announce("segment_sum large grid rounds", channels, scales)
    nodes = 70000  # past the limit for every width here (C = 8: 2 lanes per segment)
    gen = np.random.default_rng(channels)
    degrees = gen.poisson(3.0, nodes).astype(np.int64)
    degrees[::997] = 32
    degrees[5::1009] = 100
    degrees[7::4001] = 0
    case_dst = torch.from_numpy(workloads.dst_from_degrees(degrees))
    offsets = ref.segment_offsets(case_dst, nodes)
    g = torch.Generator().manual_seed(channels)
    src = torch.randn(case_dst.numel(), channels, generator=g)
    w = torch.rand(case_dst.numel(), generator=g) + 0.5 if scales else None
    s = torch.rand(nodes, generator=g) + 0.5 if scales else None
    out = kernels.segment_sum(src.to(DEV), case_dst.to(DEV), offsets.to(DEV),
                              None if w is None else w.to(DEV), None if s is None else s.to(DEV))
    assert_bitwise(out, ref.segment_sum_reference(src, case_dst, offsets, w, s), "large grid vs sequential oracle")


@pytest.mark.parametrize("channels", [3, 8, 64, 128, 256, 640])
@pytest.mark.parametrize("use_order", [False, True])
def test_segment_sum_backward_matches_autograd(channels, use_order):
    announce("segment_sum bwd", channels, use_order)
    degrees = workloads.poisson_degrees(53, 9.0, seed=channels)
    dst_sorted = torch.from_numpy(workloads.dst_from_degrees(degrees))
    if use_order:
        dst, order, offsets = _shuffled(dst_sorted, seed=3)
    else:
        dst, order, offsets = dst_sorted, None, ref.segment_offsets(dst_sorted, 53)
    gen = torch.Generator().manual_seed(channels + 1)
    src = torch.randn(dst.numel(), channels, generator=gen)
    w = torch.rand(dst.numel(), generator=gen) + 0.5
    s = torch.rand(53, generator=gen) + 0.5
    g = torch.randn(53, channels, generator=gen)
    x = src.to(DEV).requires_grad_(True)
    wd = w.to(DEV).requires_grad_(True)
    sd = s.to(DEV).requires_grad_(True)
    out = kernels.segment_sum(x, dst.to(DEV), offsets.to(DEV), wd, sd, order=None if order is None else order.to(DEV))
    grads = torch.autograd.grad(out, (x, wd, sd), g.to(DEV))
    e_src, e_w, e_s = ref.segment_sum_backward_reference(g, src, dst, offsets, w, s)
    t_src, t_w, t_s = segment_sum_backward_f64(g, src, dst, 53, w, s)
    assert_bitwise(grads[0], e_src, "grad_src")
    assert_close_scaled(grads[0], t_src, what="grad_src vs fp64 truth")
    assert_gradient(grads[1], e_w, t_w, "grad_edge_scale")
    assert_gradient(grads[2], e_s, t_s, "grad_node_scale")


def test_segment_sum_node_scale_shape_and_empty_edges_backward():
    announce("segment_sum bwd shapes")
    dst, offsets = _graph([2, 1, 3])
    src = torch.arange(12, dtype=torch.float32).reshape(6, 2) / 7
    node_scale = torch.tensor([[1.0], [2.0], [3.0]])
    x = src.to(DEV).requires_grad_(True)
    s = node_scale.to(DEV).requires_grad_(True)
    out = kernels.segment_sum(x, dst.to(DEV), offsets.to(DEV), None, s)
    g = torch.randn(3, 2)
    grad_x, grad_s = torch.autograd.grad(out, (x, s), g.to(DEV))
    assert grad_s.shape == (3, 1)
    e_src, _, e_s = ref.segment_sum_backward_reference(g, src, dst, offsets, None, node_scale.reshape(-1))
    assert_bitwise(grad_x, e_src, "grad_src")
    assert_close_scaled(grad_s.reshape(-1), e_s, what="grad_node_scale")


# ---------------------------------------------------------------------------
# segment_softmax
# ---------------------------------------------------------------------------

def test_segment_softmax_reference_case_forward_and_backward():
    announce("softmax reference case")
    dst, offsets = _graph([2, 0, 3, 1])
    gen = torch.Generator().manual_seed(0)
    logit = torch.randn(6, 16, generator=gen)
    env = torch.tensor([0.9, -0.2, 0.7, 0.0, 1.1, 0.3])
    null_logit = torch.randn(4, 16, generator=gen)
    up = torch.randn(6, 16, generator=gen)
    up_null = torch.randn(4, 16, generator=gen)
    x = logit.to(DEV).requires_grad_(True)
    e = env.to(DEV).requires_grad_(True)
    n = null_logit.to(DEV).requires_grad_(True)
    alpha, null_alpha = kernels.segment_softmax(x, e, offsets.to(DEV), n)
    grads = torch.autograd.grad((alpha, null_alpha), (x, e, n), (up.to(DEV), up_null.to(DEV)))
    e_alpha, e_null = ref.segment_softmax_reference(logit, env, dst, offsets, null_logit)
    assert_close_scaled(alpha, e_alpha, what="alpha")
    assert_close_scaled(null_alpha, e_null, what="null_alpha")
    e_gl, e_ge, e_gn = ref.segment_softmax_backward_reference(up, logit, env, dst, offsets, null_logit, up_null)
    t_gl, t_ge, t_gn = segment_softmax_backward_f64(up, logit, env, dst, 4, null_logit, up_null)
    assert_gradient(grads[0], e_gl, t_gl, "grad_logit")
    assert_gradient(grads[1], e_ge, t_ge, "grad_env")
    assert_gradient(grads[2], e_gn, t_gn, "grad_null")
    per_segment = torch.zeros(4, 16).index_add_(0, dst, alpha.detach().cpu())
    assert_close_scaled(per_segment + null_alpha.detach().cpu(), torch.ones(4, 16), what="sum to one")
    assert alpha[1].count_nonzero().item() == 0 and alpha[3].count_nonzero().item() == 0


@pytest.mark.parametrize("channels", [1, 3, 8, 16, 64, 256, 260, 640])
@pytest.mark.parametrize("null", [False, True])
@pytest.mark.parametrize("use_order", [False, True])
def test_segment_softmax_with_hubs(channels, null, use_order):
    announce("softmax", channels, null, use_order)
    # Poisson(6) segments plus hubs long enough for the block-cooperative path.
    degrees = workloads.poisson_degrees(67, 6.0, seed=channels, minimum=0, hub_fraction=0.06, hub_degree=700)
    dst_sorted = torch.from_numpy(workloads.dst_from_degrees(degrees))
    if use_order:
        dst, order, offsets = _shuffled(dst_sorted, seed=channels)
    else:
        dst, order, offsets = dst_sorted, None, ref.segment_offsets(dst_sorted, 67)
    gen = torch.Generator().manual_seed(channels + 5)
    logit = torch.randn(dst.numel(), channels, generator=gen) * 2.0
    logit.view(-1)[::97] = 40.0
    logit.view(-1)[5::89] = -40.0
    env = torch.rand(dst.numel(), generator=gen) + 0.1
    env[::13] = 0.0
    env[7::29] = -1.0
    env[11::31] = float("nan")  # masked like env <= 0: the mask is !(env > 0), csrc/segment_softmax.cpp:73
    null_logit = torch.randn(67, channels, generator=gen) if null else None
    up = torch.randn(dst.numel(), channels, generator=gen)
    up_null = torch.randn(67, channels, generator=gen) if null else None

    x = logit.to(DEV).requires_grad_(True)
    e = env.to(DEV).requires_grad_(True)
    nd = null_logit.to(DEV).requires_grad_(True) if null else None
    o = None if order is None else order.to(DEV)
    result = kernels.segment_softmax(x, e, offsets.to(DEV), nd, order=o)
    alpha = result[0] if null else result
    e_alpha, e_null = ref.segment_softmax_reference(logit, env, dst, offsets, null_logit)
    assert_close_scaled(alpha, e_alpha, what="alpha vs oracle")
    truth_alpha, truth_null = (loops.segment_softmax_loop(logit, env, dst, 67, null_logit)
                               if channels <= 16 else (None, None))
    if truth_alpha is not None:
        assert_close_scaled(alpha, truth_alpha, what="alpha vs fp64 truth")
    if null:
        assert_close_scaled(result[1], e_null, what="null_alpha")
        if truth_null is not None:
            assert_close_scaled(result[1], truth_null, what="null_alpha vs fp64 truth")
        outputs, cotangents, inputs = (result[0], result[1]), (up.to(DEV), up_null.to(DEV)), (x, e, nd)
    else:
        outputs, cotangents, inputs = (alpha,), (up.to(DEV),), (x, e)
    grads = torch.autograd.grad(outputs, inputs, cotangents)
    e_gl, e_ge, e_gn = ref.segment_softmax_backward_reference(up, logit, env, dst, offsets, null_logit, up_null)
    t_gl, t_ge, t_gn = segment_softmax_backward_f64(up, logit, env, dst, 67, null_logit, up_null)
    assert_gradient(grads[0], e_gl, t_gl, "grad_logit")
    assert_gradient(grads[1], e_ge, t_ge, "grad_env")
    if null:
        assert_gradient(grads[2], e_gn, t_gn, "grad_null")


@pytest.mark.parametrize("channels", [1, 3, 8, 16, 64, 256])
@pytest.mark.parametrize("use_order", [False, True])
def test_segment_softmax_planned_and_unplanned_paths(channels, use_order):
    """Degrees straddle every path boundary: the register path of a lane group,
    the staged and the streaming workgroup paths.  The degree plan must not
    change a single bit, and both must match the oracle."""
    from bysj_amd.kernels import _C

    announce("softmax paths", channels, use_order)
    degrees = np.array([0, 1, 5, 6, 7, 12, 13, 16, 17, 47, 48, 49, 95, 96, 97, 191, 192, 193, 255, 256, 257,
                        300, 511, 512, 513, 700, 1023, 1024, 1025, 2000, 3, 9], dtype=np.int64)
    dst_sorted = torch.from_numpy(workloads.dst_from_degrees(degrees))
    n = degrees.size
    if use_order:
        dst, order, offsets = _shuffled(dst_sorted, seed=channels)
    else:
        dst, order, offsets = dst_sorted, None, ref.segment_offsets(dst_sorted, n)
    gen = torch.Generator().manual_seed(channels)
    logit = torch.randn(dst.numel(), channels, generator=gen) * 2.0
    logit.view(-1)[::101] = 40.0
    env = torch.rand(dst.numel(), generator=gen) + 0.1
    env[::11] = -1.0
    null_logit = torch.randn(n, channels, generator=gen)
    up = torch.randn(dst.numel(), channels, generator=gen)
    up_null = torch.randn(n, channels, generator=gen)
    d_logit, d_env, d_off = logit.to(DEV), env.to(DEV), offsets.to(DEV)
    d_order = None if order is None else order.to(DEV)
    plan = _C.segment_softmax_plan(d_off, dst.numel(), channels)
    a0, n0 = _C.segment_softmax_forward(d_logit, d_env, d_off, null_logit.to(DEV), d_order)
    a1, n1 = _C.segment_softmax_forward(d_logit, d_env, d_off, null_logit.to(DEV), d_order, plan=plan)
    assert_bitwise(a1, a0, "planned alpha")
    assert_bitwise(n1, n0, "planned null_alpha")
    e_alpha, e_null = ref.segment_softmax_reference(logit, env, dst, offsets, null_logit)
    assert_close_scaled(a1, e_alpha, what="alpha")
    assert_close_scaled(n1, e_null, what="null_alpha")
    nn = _C.segment_softmax_forward(d_logit, d_env, d_off, None, d_order, plan=plan)[0]
    assert_close_scaled(nn, ref.segment_softmax_reference(logit, env, dst, offsets)[0], what="alpha without null")
    g0 = _C.segment_softmax_backward(a1, up.to(DEV), d_env, d_off, n1, up_null.to(DEV), d_order)
    g1 = _C.segment_softmax_backward(a1, up.to(DEV), d_env, d_off, n1, up_null.to(DEV), d_order, plan=plan)
    for x, y, what in zip(g1, g0, ("grad_logit", "grad_null", "grad_env")):
        assert_bitwise(x, y, f"planned {what}")
    e_gl, e_ge, e_gn = ref.segment_softmax_backward_reference(up, logit, env, dst, offsets, null_logit, up_null)
    t_gl, t_ge, t_gn = segment_softmax_backward_f64(up, logit, env, dst, n, null_logit, up_null)
    assert_gradient(g1[0], e_gl, t_gl, "grad_logit")
    assert_gradient(g1[1], e_gn, t_gn, "grad_null")
    assert_gradient(g1[2], e_ge, t_ge, "grad_env")


def test_segment_softmax_plan_lists_the_long_segments():
    from bysj_amd.kernels import _C

    announce("softmax plan")
    degrees = workloads.poisson_degrees(20000, 48.0, seed=3, hub_fraction=0.01, hub_degree=512)
    offsets = torch.from_numpy(workloads.offsets_from_degrees(degrees)).to(DEV)
    plan = _C.segment_softmax_plan(offsets, int(degrees.sum()), 8)
    words = plan.words.cpu()
    capacity = int(words[0])
    expected = np.nonzero(degrees > capacity)[0]
    assert capacity == 96 and plan.n_long == int(words[1]) == expected.size
    assert words[2:2 + plan.n_long].tolist() == expected.tolist()


def test_segment_softmax_empty_and_masked_segments():
    announce("softmax empty/masked")
    dst, offsets = _graph([0, 2, 3])
    logit = torch.randn(5, 4)
    env = torch.tensor([-1.0, 0.0, 0.5, 0.5, 0.5])  # segment 1 fully masked
    alpha = kernels.segment_softmax(logit.to(DEV), env.to(DEV), offsets.to(DEV))
    e_alpha, _ = ref.segment_softmax_reference(logit, env, dst, offsets)
    assert_close_scaled(alpha, e_alpha, what="alpha")
    assert alpha[:2].count_nonzero().item() == 0
    null_logit = torch.randn(3, 4)
    alpha, null_alpha = kernels.segment_softmax(logit.to(DEV), env.to(DEV), offsets.to(DEV), null_logit.to(DEV))
    torch.testing.assert_close(null_alpha[0].cpu(), torch.ones(4))  # null only: all mass on the null
    torch.testing.assert_close(null_alpha[1].cpu(), torch.ones(4))


@pytest.mark.parametrize("channels", [8, 64, 260])
def test_identity_order_equals_no_order(channels):
    """order = arange(E) names the natural slots: segment_sum and segment_softmax, forward and
    backward, must give the same bits as order=None on every path (short, staged and long
    segments, lane groups and wide rows)."""
    announce("identity order", channels)
    n_nodes = 300
    degrees = workloads.poisson_degrees(n_nodes, 9.0, seed=channels, minimum=0, hub_fraction=0.02,
                                        hub_degree=900)
    dst = torch.from_numpy(workloads.dst_from_degrees(degrees))
    offsets = ref.segment_offsets(dst, n_nodes).to(DEV)
    edges = dst.numel()
    identity = torch.arange(edges, dtype=torch.int64, device=DEV)
    gen = torch.Generator().manual_seed(channels)
    src = torch.randn(edges, channels, generator=gen)
    edge_scale = torch.rand(edges, generator=gen) + 0.5
    node_scale = torch.rand(n_nodes, generator=gen) + 0.5
    grad_out = torch.randn(n_nodes, channels, generator=gen)
    logit = torch.randn(edges, channels, generator=gen) * 2.0
    env = torch.rand(edges, generator=gen) + 0.1
    env[::11] = 0.0
    null_logit = torch.randn(n_nodes, channels, generator=gen)
    up = torch.randn(edges, channels, generator=gen)
    up_null = torch.randn(n_nodes, channels, generator=gen)

    def run(order):
        s, w, n = (t.to(DEV).requires_grad_(True) for t in (src, edge_scale, node_scale))
        out = kernels.segment_sum(s, dst.to(DEV), offsets, w, n, order=order)
        sum_grads = torch.autograd.grad(out, (s, w, n), grad_out.to(DEV))
        x, e, nl = (t.to(DEV).requires_grad_(True) for t in (logit, env, null_logit))
        alpha, null_alpha = kernels.segment_softmax(x, e, offsets, nl, order=order)
        soft_grads = torch.autograd.grad((alpha, null_alpha), (x, e, nl), (up.to(DEV), up_null.to(DEV)))
        return (out.detach(), *sum_grads, alpha.detach(), null_alpha.detach(), *soft_grads)

    for i, (got, want) in enumerate(zip(run(identity), run(None))):
        assert_bitwise(got, want, f"output {i}")


def test_operators_on_inference_tensors():
    """Tensors made under torch.inference_mode keep no version counter: the operators then cache
    nothing (the softmax runs without its degree plan, GIE groups on every call) and still match
    the oracle, hubs and an unsorted GIE dst included."""
    announce("inference tensors")
    n_nodes = 200
    degrees = workloads.poisson_degrees(n_nodes, 8.0, seed=3, minimum=0, hub_fraction=0.03, hub_degree=600)
    dst_cpu = torch.from_numpy(workloads.dst_from_degrees(degrees))
    offsets_cpu = ref.segment_offsets(dst_cpu, n_nodes)
    edges = dst_cpu.numel()
    gen = torch.Generator().manual_seed(3)
    logit, env = torch.randn(edges, 8, generator=gen) * 2.0, torch.rand(edges, generator=gen) + 0.1
    null_logit, src = torch.randn(n_nodes, 8, generator=gen), torch.randn(edges, 64, generator=gen)
    perm = torch.randperm(edges, generator=gen)
    zonal, radial = torch.randn(edges, 15, generator=gen), torch.randn(edges, 16, 16, generator=gen)
    slots, inv = torch.arange(1, 16), torch.rand(n_nodes, generator=gen) + 0.2
    with torch.inference_mode():
        dst, offsets = dst_cpu.to(DEV), offsets_cpu.to(DEV)
        assert offsets.is_inference()
        results = []
        for _ in range(2):
            alpha, null_alpha = kernels.segment_softmax(logit.to(DEV), env.to(DEV), offsets, null_logit.to(DEV))
            summed = kernels.segment_sum(src.to(DEV), dst, offsets)
            gie = kernels.zonal_scatter(zonal.to(DEV), radial.to(DEV), dst[perm.to(DEV)], slots.to(DEV), inv.to(DEV))
            results.append((alpha, null_alpha, summed, gie))
    e_alpha, e_null = ref.segment_softmax_reference(logit, env, dst_cpu, offsets_cpu, null_logit)
    assert_close_scaled(results[0][0], e_alpha, what="alpha")
    assert_close_scaled(results[0][1], e_null, what="null_alpha")
    assert_bitwise(results[0][2], ref.segment_sum_reference(src, dst_cpu, offsets_cpu), "segment_sum")
    assert_close_scaled(results[0][3], gie_ref.zonal_scatter_reference(zonal, radial, dst_cpu[perm], slots, inv),
                        what="zonal_scatter")
    for i, (got, want) in enumerate(zip(results[1], results[0])):
        assert_bitwise(got, want, f"second call, output {i}")


@pytest.mark.parametrize("channels", [8, 260])
def test_segment_softmax_fully_masked_long_segments(channels):
    """Hub segments whose envelopes are all <= 0 or NaN (staged and streamed long paths): alpha is
    zero there, the null logit takes all the mass, and the gradients match the oracle."""
    announce("softmax masked hubs", channels)
    dst, offsets = _graph([5, 700, 3, 5000, 0, 2])
    edges = dst.numel()
    gen = torch.Generator().manual_seed(channels)
    logit = torch.randn(edges, channels, generator=gen) * 2.0
    env = torch.rand(edges, generator=gen) + 0.1
    env[5:705] = -0.5
    env[708:5708] = 0.0
    env[708:5708:7] = float("nan")
    up = torch.randn(edges, channels, generator=gen)
    for null in (False, True):
        null_logit = torch.randn(6, channels, generator=gen) if null else None
        up_null = torch.randn(6, channels, generator=gen) if null else None
        x, e = logit.to(DEV).requires_grad_(True), env.to(DEV).requires_grad_(True)
        nd = null_logit.to(DEV).requires_grad_(True) if null else None
        result = kernels.segment_softmax(x, e, offsets.to(DEV), nd)
        alpha = result[0] if null else result
        e_alpha, e_null = ref.segment_softmax_reference(logit, env, dst, offsets, null_logit)
        assert_close_scaled(alpha, e_alpha, what=f"alpha (null={null})")
        assert alpha[5:705].count_nonzero().item() == 0 and alpha[708:5708].count_nonzero().item() == 0
        if null:
            torch.testing.assert_close(result[1][1].cpu(), torch.ones(channels))
            torch.testing.assert_close(result[1][3].cpu(), torch.ones(channels))
            outputs, cotangents, inputs = (result[0], result[1]), (up.to(DEV), up_null.to(DEV)), (x, e, nd)
        else:
            outputs, cotangents, inputs = (alpha,), (up.to(DEV),), (x, e)
        grads = torch.autograd.grad(outputs, inputs, cotangents)
        e_gl, e_ge, e_gn = ref.segment_softmax_backward_reference(up, logit, env, dst, offsets, null_logit, up_null)
        t_gl, t_ge, t_gn = segment_softmax_backward_f64(up, logit, env, dst, 6, null_logit, up_null)
        assert_gradient(grads[0], e_gl, t_gl, "grad_logit")
        assert_gradient(grads[1], e_ge, t_ge, "grad_env")
        assert grads[1][5:705].count_nonzero().item() == 0 and grads[1][708:5708].count_nonzero().item() == 0
        if null:
            assert_gradient(grads[2], e_gn, t_gn, "grad_null")


def test_segment_softmax_config2_full_size_and_determinism():
    announce("softmax config 2")
    case = workloads.segment_softmax_config(seed=0)
    d = {k: (v.to(DEV) if v is not None else None) for k, v in case.items()}
    alpha, null_alpha = kernels.segment_softmax(d["logit"], d["env"], d["offsets"], d["null_logit"])
    again, again_null = kernels.segment_softmax(d["logit"], d["env"], d["offsets"], d["null_logit"])
    assert_bitwise(alpha, again, "run-to-run alpha")
    assert_bitwise(null_alpha, again_null, "run-to-run null")
    e_alpha, e_null = ref.segment_softmax_reference(case["logit"], case["env"], case["dst"], case["offsets"],
                                                    case["null_logit"])
    assert_close_scaled(alpha, e_alpha, what="config 2 alpha")
    assert_close_scaled(null_alpha, e_null, what="config 2 null_alpha")
    total = torch.zeros_like(null_alpha).index_add_(0, d["dst"], alpha) + null_alpha
    assert_close_scaled(total, torch.ones_like(total), what="sum to one")


# ---------------------------------------------------------------------------
# force_assembly
# ---------------------------------------------------------------------------

def test_force_assembly_reference_case():
    announce("force reference case")
    dst, dst_offsets = _graph([2, 1, 3, 0])
    src = torch.tensor([2, 0, 2, 1, 0, 2], dtype=torch.int64)
    gen = torch.Generator().manual_seed(0)
    g = torch.randn(6, 3, generator=gen)
    v = torch.randn(6, 3, generator=gen)
    force, virial = kernels.force_assembly(g.to(DEV), v.to(DEV), src.to(DEV), dst.to(DEV), dst_offsets.to(DEV))
    order, src_offsets = ref.group_by_source(src, 4)
    e_force, e_virial = ref.force_assembly_reference(g, v, src, dst, dst_offsets, src_offsets)
    truth_force, truth_virial = loops.force_assembly_loop(g, v, src, dst, 4)
    assert_close_scaled(force, e_force, what="force vs oracle")
    assert_close_scaled(virial, e_virial, what="virial vs oracle")
    assert_close_scaled(force, truth_force, what="force vs fp64 truth")
    assert_close_scaled(virial, truth_virial, what="virial vs fp64 truth")
    assert force[3].count_nonzero().item() == 0


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_force_assembly_grouped_graph(dtype):
    announce("force grouped", dtype)
    gen = torch.Generator().manual_seed(7)
    atoms, edges = 64, 4096
    dst = torch.sort(torch.randint(0, atoms, (edges,), generator=gen)).values
    offsets = ref.segment_offsets(dst, atoms)
    src = torch.randint(0, atoms, (edges,), generator=gen)
    order, src_offsets = ref.group_by_source(src, atoms)
    g = torch.randn(edges, 3, generator=gen, dtype=torch.float64).to(dtype)
    v = torch.randn(edges, 3, generator=gen, dtype=torch.float64).to(dtype)
    force, virial = kernels.force_assembly(g.to(DEV), v.to(DEV), src.to(DEV), dst.to(DEV), offsets.to(DEV),
                                           src_offsets.to(DEV), order.to(DEV))
    assert force.dtype == dtype and virial.dtype == dtype
    truth_force, truth_virial = loops.force_assembly_loop(g, v, src, dst, atoms)
    if dtype == torch.float64:
        assert_fp64(force, truth_force, "fp64 force")
        assert_fp64(virial, truth_virial, "fp64 virial")
        assert abs(float(force.sum(0).abs().max())) <= 1e-12 * float(g.abs().sum())
    else:
        e_force, e_virial = ref.force_assembly_reference(g, v, src, dst, offsets, src_offsets)
        assert_close_scaled(force, e_force, what="force vs oracle")
        assert_close_scaled(virial, e_virial, what="virial vs oracle")
        assert_close_scaled(force, truth_force, what="force vs truth")
        assert_close_scaled(virial, truth_virial, what="virial vs truth")


def test_force_assembly_water_graph_newton_and_determinism():
    announce("force water graph")
    graph = workloads.water_graph(2048, seed=3)
    case = workloads.force_config(graph, seed=3, device="cpu", dtype=torch.float64)
    d = {k: v.to(DEV) for k, v in case.items()}
    force, virial = kernels.force_assembly(d["grad_edge"], d["edge_vec"], d["src"], d["dst"], d["dst_offsets"],
                                           d["src_offsets"], d["src_order"])
    again, again_virial = kernels.force_assembly(d["grad_edge"], d["edge_vec"], d["src"], d["dst"],
                                                 d["dst_offsets"], d["src_offsets"], d["src_order"])
    assert_bitwise(force, again, "run-to-run force")
    assert_bitwise(virial, again_virial, "run-to-run virial")
    e_force, e_virial = ref.force_assembly_reference(case["grad_edge"], case["edge_vec"], case["src"], case["dst"],
                                                     case["dst_offsets"], case["src_offsets"])
    assert_fp64(force, e_force, "fp64 force vs oracle")
    assert_fp64(virial, e_virial, "fp64 virial vs oracle")
    net = force.sum(0).abs().max().item()
    assert net <= 1e-12 * case["grad_edge"].abs().sum().item()
