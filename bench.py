#!/usr/bin/env python3
"""Benchmark of the MI355X DPA4/SeZM operator slice (one GPU).

Headline: segment_softmax forward with the null
logit, N = 16,384 nodes (1 % hubs of degree 512, rest Poisson(48)),
E ~ 862k edges, C = 8 heads, fp32.  A *step* is one forward pass over one
batch of that shape.  The job cycles through enough distinct input batches
(same graph, fresh logits / envelopes / null logits) that their total size
exceeds the 256 MB Infinity Cache several times over, so every step streams
its inputs from HBM.  The K timed steps are captured once into a HIP graph
and replayed between two HIP events on the capturing stream; warmup steps run
eagerly first.  `value` is edges per second over the K steps.

The `roofline` object prices the same timed region: algorithmic bytes of one
launch (every input read once, every output written once) over the average
duration per launch.  `cpu_baseline` times the CPU oracle (the reference's
ATen chain restated in torch) on the host cores on a bounded sample.  `ops`
repeats the measurement for the other operators at their configuration sizes.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--headline-only]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBPS = 8000.0
MALL_BYTES = 256 * 2**20
ROTATION_BYTES = 1 << 30  # distinct input bytes cycled through per op
TRAFFIC_FILE = ROOT / "profiles" / "traffic.json"


def parse_args():
    parser = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=200)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--headline-only", action="store_true", help="skip the per-operator lines")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-backward", action="store_true", help="skip the backward and CSR-build lines")
    parser.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline sample length")
    parser.add_argument("--eager", action="store_true", help="time eager launches instead of a graph replay")
    parser.add_argument("--roofline-shapes", action="store_true",
                        help="also run the >=10M-edge shapes (1R, 2R, 4R)")
    parser.add_argument("--calibrate-copy", action="store_true",
                        help="launch one plain 256 MiB copy (counter calibration for rocprofv3 --pmc)")
    return parser.parse_args()


# ---------------------------------------------------------------------------
# timing harness
# ---------------------------------------------------------------------------

def time_steps(step, n_sets: int, steps: int, warmup: int, *, graph: bool = True) -> float:
    """Average milliseconds per step over `steps` steps (step(i) uses input set i % n_sets)."""
    import torch

    for i in range(warmup):
        step(i % n_sets)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    if graph:
        hip_graph = torch.cuda.CUDAGraph()
        keep = []
        with torch.cuda.graph(hip_graph):
            for i in range(steps):
                keep.append(step(i % n_sets))
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        hip_graph.replay()
        stop.record(stream)
        torch.cuda.synchronize()
        elapsed = start.elapsed_time(stop)
        del keep, hip_graph
    else:
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for i in range(steps):
            step(i % n_sets)
        stop.record(stream)
        torch.cuda.synchronize()
        elapsed = start.elapsed_time(stop)
    return elapsed / steps


def n_sets_for(bytes_per_set: int) -> int:
    return max(1, min(64, -(-ROTATION_BYTES // max(1, bytes_per_set))))


def measured_traffic(key: str | None, bytes_per_launch: int) -> int | None:
    """HBM bytes per launch from the committed FETCH_SIZE + WRITE_SIZE summary, when it is for this workload.

    profiles/traffic.json holds the calibrated counter totals of one rocprofv3 --pmc pass per
    counter for every bench line (the headline and each entry of `ops`); an entry counts only when
    its algorithmic byte total equals this run's, so a changed workload reports null instead of a
    stale figure.
    """
    if key is None:
        return None
    try:
        entry = json.loads(TRAFFIC_FILE.read_text())[key]
    except (OSError, ValueError, KeyError):
        return None
    if int(entry.get("algorithmic_bytes", -1)) != int(bytes_per_launch):
        return None
    return int(entry["bytes_per_launch"])


def roofline(bytes_per_launch: int, ms_per_launch: float, traffic_key: str | None = None) -> dict:
    achieved = bytes_per_launch / (ms_per_launch * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": measured_traffic(traffic_key, bytes_per_launch),
            "algorithmic_bytes": int(bytes_per_launch)}


def cpu_time(function, seconds: float) -> tuple[float, int]:
    """Median seconds per call of `function` over about `seconds` of work (after 2 warmups)."""
    for _ in range(2):
        function()
    samples = []
    begin = time.perf_counter()
    while len(samples) < 5 or (time.perf_counter() - begin < seconds and len(samples) < 1000):
        t0 = time.perf_counter()
        function()
        samples.append(time.perf_counter() - t0)
    samples.sort()
    return samples[len(samples) // 2], len(samples)


# ---------------------------------------------------------------------------
# workloads
# ---------------------------------------------------------------------------

def softmax_job(n_nodes: int, steps: int, warmup: int, graph: bool):
    import torch

    from bysj_amd import kernels, workloads

    base = workloads.segment_softmax_config(n_nodes=n_nodes, seed=0, device="cuda")
    edges, channels = base["logit"].shape
    offsets = base["offsets"]
    bytes_per_step = 2 * edges * channels * 4 + edges * 4 + (n_nodes + 1) * 8 + 2 * n_nodes * channels * 4
    n_sets = n_sets_for(bytes_per_step)
    # one graph; every input set draws fresh logits, envelopes and null logits
    sets = [base] + [workloads.segment_softmax_features(edges, n_nodes, channels, seed=s, device="cuda")
                     for s in range(1, n_sets)]

    def step(i):
        case = sets[i]
        return kernels.segment_softmax(case["logit"], case["env"], offsets, case["null_logit"])

    with torch.no_grad():
        ms = time_steps(step, n_sets, steps, warmup, graph=graph)
    return {"edges": int(edges), "nodes": n_nodes, "channels": int(channels), "sets": n_sets,
            "ms_per_step": ms, "bytes": bytes_per_step, "base": base}


def segment_sum_job(n_nodes: int, steps: int, warmup: int, graph: bool, scaled_shuffled: bool = False):
    """segment_sum forward; `scaled_shuffled` adds edge and node scales ~U(0.5, 1.5) and a shuffled edge order."""
    import torch

    from bysj_amd import kernels, workloads

    base = workloads.segment_sum_config(n_nodes=n_nodes, seed=0, device="cuda")
    edges, channels = base["src"].shape
    bytes_per_step = edges * channels * 4 + (n_nodes + 1) * 8 + n_nodes * channels * 4
    generator = torch.Generator(device="cuda")
    generator.manual_seed(1)
    dst, edge_scale, node_scale, order = base["dst"], None, None, None
    if scaled_shuffled:
        edge_scale = torch.rand(edges, generator=generator, device="cuda") + 0.5
        node_scale = torch.rand(n_nodes, generator=generator, device="cuda") + 0.5
        order = torch.randperm(edges, generator=generator, device="cuda")  # slot i holds edge order[i]
        dst = torch.empty_like(base["dst"])
        dst[order] = base["dst"]
        bytes_per_step += edges * 4 + n_nodes * 4 + edges * 8
    n_sets = n_sets_for(bytes_per_step)
    sets = [base["src"]] + [torch.randn(base["src"].shape, generator=generator, device="cuda")
                            for _ in range(1, n_sets)]

    def step(i):
        return kernels.segment_sum(sets[i], dst, base["offsets"], edge_scale, node_scale, order=order)

    with torch.no_grad():
        ms = time_steps(step, n_sets, steps, warmup, graph=graph)
    return {"edges": int(edges), "nodes": n_nodes, "channels": int(channels), "sets": n_sets,
            "ms_per_step": ms, "bytes": bytes_per_step, "base": base}


def gie_rmsnorm_jobs(n_atoms: int, steps: int, warmup: int, graph: bool, water=None, gie_steps=None):
    import torch

    from bysj_amd import workloads
    from bysj_amd.kernels import _C

    water = water or workloads.water_graph(n_atoms, seed=0)
    case = workloads.gie_config(water, seed=0, device="cuda", primary=True)
    edges = water.n_edges
    offsets, order, _ = _C.gie_group(case["dst"], case["radial_slot"], n_atoms, 16)

    def gie_step(_):
        return _C.gie_zonal_scatter_forward_csr(case["zonal"], case["radial"], offsets, order,
                                                case["radial_slot"], case["inv_sqrt_deg"])

    gie_bytes = edges * 15 * 4 + edges * 15 * 64 * 4 + (n_atoms + 1) * 8 + 15 * 8 + n_atoms * 4 \
        + n_atoms * 16 * 64 * 4
    width = 16 * 64
    fused_bytes = gie_bytes - n_atoms * width * 4 + n_atoms * width * 4 + width * 4 + n_atoms * 4

    def fused_step(_):
        return _C.gie_rmsnorm_forward_csr(case["zonal"], case["radial"], offsets, order, case["radial_slot"],
                                          case["inv_sqrt_deg"], case["rms_scale"], 1e-6, False)

    with torch.no_grad():
        gie_ms = time_steps(gie_step, 1, gie_steps or max(4, steps // 10), min(warmup, 3), graph=graph)
        fused_ms = time_steps(fused_step, 1, gie_steps or max(4, steps // 10), min(warmup, 3), graph=graph)
        rows = gie_step(0).reshape(n_atoms, 1024)
    rms_bytes = 2 * n_atoms * 1024 * 4 + 1024 * 4 + n_atoms * 4
    n_sets = n_sets_for(rms_bytes)
    generator = torch.Generator(device="cuda")
    generator.manual_seed(3)
    row_sets = [rows] + [torch.randn(rows.shape, generator=generator, device="cuda") for _ in range(1, n_sets)]

    def rms_step(i):
        return _C.rmsnorm_forward(row_sets[i], case["rms_scale"], 1e-6)

    with torch.no_grad():
        rms_ms = time_steps(rms_step, n_sets, steps, warmup, graph=graph)
    gie = {"edges": edges, "nodes": n_atoms, "ms_per_step": gie_ms, "bytes": gie_bytes, "sets": 1}
    rms = {"rows": n_atoms, "width": 1024, "ms_per_step": rms_ms, "bytes": rms_bytes, "sets": n_sets}
    gie["fused_rmsnorm"] = {"edges": edges, "nodes": n_atoms, "ms_per_step": fused_ms, "bytes": fused_bytes,
                            "sets": 1}
    return gie, rms, water, case


def force_job(n_atoms: int, steps: int, warmup: int, graph: bool, dtype_name: str, water=None):
    import torch

    from bysj_amd import kernels, workloads

    dtype = torch.float32 if dtype_name == "f32" else torch.float64
    water = water or workloads.water_graph(n_atoms, seed=0)
    base = workloads.force_config(water, seed=0, device="cuda", dtype=dtype)
    edges = water.n_edges
    size = 4 if dtype == torch.float32 else 8
    bytes_per_step = 2 * edges * 3 * size + edges * 8 + 2 * (n_atoms + 1) * 8 + n_atoms * 12 * size
    n_sets = n_sets_for(bytes_per_step)
    generator = torch.Generator(device="cuda")
    generator.manual_seed(5)
    # every set has its own gradients and edge vectors (the same geometry, jittered): each step reads
    # both from HBM; the graph (offsets, src_order) is fixed, as within one neighbour-list lifetime
    sets = [(base["grad_edge"], base["edge_vec"])] + [
        (torch.randn(base["grad_edge"].shape, generator=generator, device="cuda", dtype=dtype),
         base["edge_vec"] + 0.01 * torch.randn(base["edge_vec"].shape, generator=generator, device="cuda",
                                               dtype=dtype))
        for _ in range(1, n_sets)]

    def step(i):
        grad_edge, edge_vec = sets[i]
        return kernels.force_assembly(grad_edge, edge_vec, base["src"], base["dst"], base["dst_offsets"],
                                      base["src_offsets"], base["src_order"])

    with torch.no_grad():
        ms = time_steps(step, n_sets, steps, warmup, graph=graph)
    return {"edges": edges, "nodes": n_atoms, "ms_per_step": ms, "bytes": bytes_per_step, "sets": n_sets,
            "dtype": dtype_name}, water, base


def softmax_backward_job(n_nodes: int, steps: int, warmup: int, graph: bool):
    """segment_softmax backward (with the null logit) on the config-2 graph.

    Every input set holds its own alpha, null alpha (forward outputs of fresh logits), envelope
    and cotangents, so each step reads them from HBM.
    """
    import torch

    from bysj_amd import kernels, workloads
    from bysj_amd.kernels import _C

    base = workloads.segment_softmax_config(n_nodes=n_nodes, seed=0, device="cuda")
    edges, channels = base["logit"].shape
    offsets = base["offsets"]
    plan = _C.segment_softmax_plan(offsets, edges, channels)
    reads = 2 * edges * channels * 4 + edges * 4 + (n_nodes + 1) * 8 + 2 * n_nodes * channels * 4
    writes = edges * channels * 4 + n_nodes * channels * 4 + edges * 4
    n_sets = n_sets_for(reads + writes)
    generator = torch.Generator(device="cuda")
    generator.manual_seed(7)
    sets = []
    for s in range(n_sets):
        features = base if s == 0 else workloads.segment_softmax_features(edges, n_nodes, channels, seed=s,
                                                                          device="cuda")
        with torch.no_grad():
            alpha, null_alpha = kernels.segment_softmax(features["logit"], features["env"], offsets,
                                                        features["null_logit"])
        sets.append((alpha, null_alpha, features["env"], torch.randn(alpha.shape, generator=generator, device="cuda"),
                     torch.randn(null_alpha.shape, generator=generator, device="cuda")))
        del features

    def step(i):
        alpha, null_alpha, env, grad_alpha, grad_null = sets[i]
        return _C.segment_softmax_backward(alpha, grad_alpha, env, offsets, null_alpha, grad_null, plan=plan)

    ms = time_steps(step, n_sets, steps, warmup, graph=graph)
    return {"edges": int(edges), "nodes": n_nodes, "channels": int(channels), "sets": n_sets, "ms_per_step": ms,
            "bytes": reads + writes}


def segment_sum_backward_job(n_nodes: int, steps: int, warmup: int, graph: bool):
    """segment_sum backward with edge_scale and node_scale: grad_src, grad_edge_scale, grad_node_scale.

    Every input set holds its own src, scales and grad_out, so each step reads them from HBM.
    """
    import torch

    from bysj_amd import workloads
    from bysj_amd.kernels import _C

    base = workloads.segment_sum_config(n_nodes=n_nodes, seed=0, device="cuda", scales=True)
    edges, channels = base["src"].shape
    reads = n_nodes * channels * 4 + edges * channels * 4 + edges * 4 + n_nodes * 4 + (n_nodes + 1) * 8
    writes = edges * channels * 4 + edges * 4 + n_nodes * 4
    n_sets = n_sets_for(reads + writes)
    generator = torch.Generator(device="cuda")
    generator.manual_seed(8)
    sets = []
    for s in range(n_sets):
        src = base["src"] if s == 0 else torch.randn(base["src"].shape, generator=generator, device="cuda")
        edge_scale = torch.rand(edges, generator=generator, device="cuda") + 0.5
        node_scale = torch.rand(n_nodes, generator=generator, device="cuda") + 0.5
        grad = torch.randn((n_nodes, channels), generator=generator, device="cuda")
        sets.append((grad, src, edge_scale, node_scale))

    def step(i):
        grad, src, edge_scale, node_scale = sets[i]
        return _C.segment_sum_backward(grad, src, base["dst"], base["offsets"], edge_scale, node_scale, True, None,
                                       want_edge_scale_grad=True)

    ms = time_steps(step, n_sets, steps, warmup, graph=graph)
    return {"edges": int(edges), "nodes": n_nodes, "channels": int(channels), "sets": n_sets, "ms_per_step": ms,
            "bytes": reads + writes}


def gie_rmsnorm_backward_jobs(water, case, steps: int, warmup: int, graph: bool, gie_steps=None):
    """GIE backward (zonal, radial and inverse-degree gradients) and RMSNorm backward on a water box."""
    import torch

    from bysj_amd.kernels import _C

    n_atoms, edges = water.n_atoms, water.n_edges
    offsets, order, info = _C.gie_group(case["dst"], case["radial_slot"], n_atoms, 16)
    generator = torch.Generator(device="cuda")
    generator.manual_seed(9)
    grad_out = torch.randn((n_atoms, 16, 64), generator=generator, device="cuda")

    def gie_step(_):
        return _C.gie_zonal_scatter_backward_csr(grad_out, case["zonal"], case["radial"], offsets, order,
                                                 case["radial_slot"], case["inv_sqrt_deg"], bool(info & 2))

    gie_reads = n_atoms * 15 * 64 * 4 + edges * 15 * 4 + edges * 15 * 64 * 4 + (n_atoms + 1) * 8 + 15 * 8 \
        + n_atoms * 4
    gie_writes = edges * 15 * 4 + edges * 16 * 64 * 4 + n_atoms * 4
    gie_ms = time_steps(gie_step, 1, gie_steps or max(4, steps // 10), min(warmup, 3), graph=graph)
    del grad_out

    rms_bytes = 3 * n_atoms * 1024 * 4 + 2 * 1024 * 4 + n_atoms * 4
    n_sets = n_sets_for(rms_bytes)
    rms_sets = []
    for _ in range(n_sets):
        x = torch.randn((n_atoms, 1024), generator=generator, device="cuda")
        _, inverse_rms = _C.rmsnorm_forward(x, case["rms_scale"], 1e-6)
        rms_sets.append((torch.randn((n_atoms, 1024), generator=generator, device="cuda"), x, inverse_rms))

    def rms_step(i):
        grad, x, inverse_rms = rms_sets[i]
        return _C.rmsnorm_backward(grad, x, case["rms_scale"], inverse_rms, True)

    rms_ms = time_steps(rms_step, n_sets, steps, warmup, graph=graph)
    gie = {"edges": edges, "nodes": n_atoms, "ms_per_step": gie_ms, "bytes": gie_reads + gie_writes, "sets": 1}
    rms = {"rows": n_atoms, "width": 1024, "ms_per_step": rms_ms, "bytes": rms_bytes, "sets": n_sets}
    return gie, rms


def rmsnorm_jobs(rows: int, steps: int, warmup: int, graph: bool):
    """RMSNorm forward and backward over `rows` random rows of width 1024 (eps 1e-6, scale ~U(0.5, 1.5))."""
    import torch

    from bysj_amd.kernels import _C

    generator = torch.Generator(device="cuda")
    generator.manual_seed(13)
    scale = torch.rand(1024, generator=generator, device="cuda") + 0.5
    fwd_bytes = 2 * rows * 1024 * 4 + 1024 * 4 + rows * 4
    bwd_bytes = 3 * rows * 1024 * 4 + 2 * 1024 * 4 + rows * 4
    n_sets = n_sets_for(bwd_bytes)
    sets = []
    for _ in range(n_sets):
        x = torch.randn((rows, 1024), generator=generator, device="cuda")
        _, inverse_rms = _C.rmsnorm_forward(x, scale, 1e-6)
        sets.append((x, inverse_rms, torch.randn((rows, 1024), generator=generator, device="cuda")))
    with torch.no_grad():
        fwd_ms = time_steps(lambda i: _C.rmsnorm_forward(sets[i][0], scale, 1e-6), n_sets, steps, warmup, graph=graph)
    bwd_ms = time_steps(lambda i: _C.rmsnorm_backward(sets[i][2], sets[i][0], scale, sets[i][1], True), n_sets,
                        steps, warmup, graph=graph)
    fwd = {"rows": rows, "width": 1024, "ms_per_step": fwd_ms, "bytes": fwd_bytes, "sets": n_sets}
    bwd = {"rows": rows, "width": 1024, "ms_per_step": bwd_ms, "bytes": bwd_bytes, "sets": n_sets}
    return fwd, bwd


def csr_job(water, steps: int, warmup: int, graph: bool):
    """Device CSR build of a source list (group_by_source: offsets + stable order) on the config-4 graph.

    The step is the asynchronous build (_C.group_by_key_async: every kernel of the counting sort, no
    host round trip) on buffers allocated once, timed like the other lines, on source lists that
    rotate through enough distinct permutations of the graph's `src` to leave the Infinity Cache.
    `eager_ms_per_call` times kernels.group_by_source itself (allocations, the Python layer and the
    host synchronisation of its range check), and `torch_argsort_bincount_ms` the PyTorch chain.
    """
    import torch

    from bysj_amd import kernels
    from bysj_amd.kernels import _C, _lib

    src = torch.from_numpy(water.src).to("cuda")
    n_atoms, edges = water.n_atoms, water.n_edges
    bytes_per_step = edges * 8 + edges * 8 + (n_atoms + 1) * 8
    n_sets = n_sets_for(bytes_per_step)
    generator = torch.Generator(device="cuda")
    generator.manual_seed(17)
    sets = [src] + [src[torch.randperm(edges, generator=generator, device="cuda")] for _ in range(1, n_sets)]
    buffers = [dict(order=torch.empty(edges, dtype=torch.int64, device="cuda"),
                    offsets=torch.empty(n_atoms + 1, dtype=torch.int64, device="cuda"),
                    status=torch.zeros(1, dtype=torch.int32, device="cuda")) for _ in range(n_sets)]
    workspace = torch.empty(_lib.load().dpa4k_group_by_key_workspace_size(edges, n_atoms), dtype=torch.uint8,
                            device="cuda")
    ms = time_steps(lambda i: _C.group_by_key_async(sets[i], n_atoms, workspace=workspace, **buffers[i]), n_sets,
                    steps, warmup, graph=graph)
    statuses = [int(b["status"].item()) for b in buffers]
    if any(code & 1 for code in statuses):
        raise RuntimeError(f"group_by_key_async reported out-of-range keys: {statuses}")
    eager_ms = time_steps(lambda _: kernels.group_by_source(src, n_atoms), 1, max(5, steps // 4), 2, graph=False)
    torch_ms = time_steps(lambda _: (torch.argsort(src, stable=True),
                                     torch.bincount(src, minlength=n_atoms).cumsum(0)), 1, max(5, steps // 4), 2,
                          graph=False)
    return {"edges": edges, "nodes": n_atoms, "ms_per_step": ms, "bytes": bytes_per_step, "sets": n_sets,
            "eager_ms_per_call": eager_ms, "torch_ms_per_call": torch_ms}


def stream_ceilings(read_bytes: int, write_bytes: int, steps: int) -> dict:
    """Read-only and copy rates of plain streams on this part, and a copy of one operator's bytes.

    1 GiB read-only and copy passes (dpa4k_stream_calibrate: grid-stride, four 16-byte chunks per
    thread per round), then a copy that reads `read_bytes` and writes `write_bytes`, rotated
    through 1 GiB of distinct sources like the operator lines.  Same graph-replay timing.
    """
    import torch

    from bysj_amd.kernels import _lib

    library = _lib.load()
    floats = 256 * 2**20
    source = torch.randn(floats, device="cuda")
    target = torch.empty(floats, device="cuda")
    sink = torch.empty(8192, device="cuda")

    def launch(src, read_floats, dst, write_floats):
        status = library.dpa4k_stream_calibrate(src.data_ptr(), read_floats, dst.data_ptr(), write_floats,
                                                torch.cuda.current_stream().cuda_stream)
        _lib.check(status)

    read_ms = time_steps(lambda _: launch(source, floats, sink, 0), 1, 10, 2)
    copy_ms = time_steps(lambda _: launch(source, floats, target, floats), 1, 10, 2)
    del source, target
    read_floats = (read_bytes // 4 + 3) // 4 * 4
    write_floats = min(read_floats, (write_bytes // 4 + 3) // 4 * 4)
    n_sets = n_sets_for(read_bytes + write_bytes)
    sources = [torch.randn(read_floats, device="cuda") for _ in range(n_sets)]
    out = torch.empty(max(write_floats, 8192), device="cuda")
    op_ms = time_steps(lambda i: launch(sources[i], read_floats, out, write_floats), n_sets, steps, 20)
    moved = (read_floats + write_floats) * 4
    return {"read_GBps": round(floats * 4 / (read_ms * 1e-3) / 1e9, 1),
            "copy_GBps": round(2 * floats * 4 / (copy_ms * 1e-3) / 1e9, 1),
            "same_bytes_copy_us": round(op_ms * 1e3, 3),
            "same_bytes_copy_GBps": round(moved / (op_ms * 1e-3) / 1e9, 1),
            "note": "plain HIP streams on this part (1 GiB read, 1 GiB copy, and a copy of the headline's "
                    "read/write bytes); the headline's ms_per_step over same_bytes_copy_us is its share of "
                    "what a stream of its own bytes reaches"}


def _torch_softmax_chain(logit, env, dst, n_nodes, null_logit):
    """The reference's PyTorch chain for segment_softmax (python/reference/segment.py:84-118), run on the GPU."""
    import torch

    valid = (env > 0).unsqueeze(1)
    eff = torch.where(valid, logit + 2.0 * torch.log(env.clamp_min(1e-30)).unsqueeze(1),
                      torch.full_like(logit, float("-inf")))
    peak = torch.full((n_nodes, logit.shape[1]), float("-inf"), device=logit.device)
    peak = peak.scatter_reduce(0, dst.unsqueeze(1).expand_as(eff), eff, reduce="amax", include_self=True)
    peak = torch.maximum(peak, null_logit)
    weight = torch.where(valid, torch.exp(eff - peak[dst]), torch.zeros_like(eff))
    null_weight = torch.exp(null_logit - peak)
    total = torch.zeros_like(peak).index_add_(0, dst, weight) + null_weight
    return weight / total[dst], null_weight / total


def _torch_force_chain(grad_edge, edge_vec, src, dst, n_nodes):
    """The reference's PyTorch chain for force_assembly (python/reference/segment.py:121-142), run on the GPU."""
    import torch

    force = torch.zeros((n_nodes, 3), device=grad_edge.device).index_add_(0, dst, grad_edge)
    force.index_add_(0, src, -grad_edge)
    outer = -(grad_edge.unsqueeze(2) * edge_vec.unsqueeze(1)).reshape(-1, 9)
    return force, torch.zeros((n_nodes, 9), device=grad_edge.device).index_add_(0, src, outer)


def _torch_sum_chain(rows, dst, n_nodes, node_scale):
    """The reference's PyTorch chain for segment_sum (python/reference/segment.py:39-60), run on the GPU."""
    import torch

    out = torch.zeros((n_nodes, rows.shape[1]), device=rows.device).index_add_(0, dst, rows)
    return out * node_scale.unsqueeze(1)


def reference_shapes(steps: int) -> dict:
    """The reference's own latency-test shapes, timed like its harnesses and as kernels.

    tests/csrc/latency/test_segment_ops_latency.py of the reference: 3,000 atoms, 181,838 edges,
    dst = sorted uniform draws, env ~ U(0.1, 1.1), logits/null logits ~ N(0, 1) at 64 and 256
    channels, force assembly on uniform random sources.  `eager_ms` follows its `_median_ms`
    (10 warmup calls, median of 5 repeats of 20 calls between events, same inputs every call);
    `kernel_ms` is the graph replay of this file.  `dcu_ms` is the reference's published figure
    on its Hygon DCU (docs/task2-hip-fusion-plan.md:229, :272), other hardware.
    """
    import torch

    from bysj_amd import kernels

    atoms, edges = 3000, 181838
    generator = torch.Generator(device="cuda")
    generator.manual_seed(11)
    dst = torch.sort(torch.randint(0, atoms, (edges,), generator=generator, device="cuda")).values
    offsets = kernels.segment_offsets(dst, atoms)
    env = torch.rand(edges, generator=generator, device="cuda") + 0.1

    def median_eager(function) -> float:
        for _ in range(10):
            function()
        torch.cuda.synchronize()
        samples = []
        for _ in range(5):
            start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            for _ in range(20):
                function()
            stop.record()
            torch.cuda.synchronize()
            samples.append(start.elapsed_time(stop) / 20)
        samples.sort()
        return samples[2]

    out = {}
    with torch.no_grad():
        # dcu_ms / dcu_torch_ms: the reference's fused operator and its PyTorch chain on its DCU;
        # torch_gpu_ms: that PyTorch chain on this GPU, timed like the fused operator
        for channels, dcu, dcu_torch in ((64, 0.49, 4.42), (256, 1.91, 9.52)):
            logit = torch.randn(edges, channels, generator=generator, device="cuda")
            null = torch.randn(atoms, channels, generator=generator, device="cuda")
            call = lambda _=None, logit=logit, null=null: kernels.segment_softmax(logit, env, offsets, null)
            chain = lambda _=None, logit=logit, null=null: _torch_softmax_chain(logit, env, dst, atoms, null)
            out[f"segment_softmax_C{channels}_null"] = {
                "eager_ms": round(median_eager(call), 4), "kernel_ms": round(time_steps(call, 1, steps, 10), 4),
                "torch_gpu_ms": round(median_eager(chain), 4), "dcu_ms": dcu, "dcu_torch_ms": dcu_torch,
                "source": "docs/task2-hip-fusion-plan.md:229"}
        src = torch.randint(0, atoms, (edges,), generator=generator, device="cuda")
        src_order, src_offsets = kernels.group_by_source(src, atoms)
        grad_edge = torch.randn(edges, 3, generator=generator, device="cuda")
        edge_vec = torch.randn(edges, 3, generator=generator, device="cuda")
        call = lambda _=None: kernels.force_assembly(grad_edge, edge_vec, src, dst, offsets, src_offsets, src_order)
        chain = lambda _=None: _torch_force_chain(grad_edge, edge_vec, src, dst, atoms)
        out["force_assembly_f32"] = {"eager_ms": round(median_eager(call), 4),
                                     "kernel_ms": round(time_steps(call, 1, steps, 10), 4),
                                     "torch_gpu_ms": round(median_eager(chain), 4), "dcu_ms": 0.182,
                                     "dcu_torch_ms": 1.006, "source": "docs/task2-hip-fusion-plan.md:272"}
        node_scale = torch.rand(atoms, generator=generator, device="cuda") + 0.5
        for channels in (64, 256):
            src_rows = torch.randn(edges, channels, generator=generator, device="cuda")
            call = lambda _=None, rows=src_rows: kernels.segment_sum(rows, dst, offsets, None, node_scale)
            chain = lambda _=None, rows=src_rows: _torch_sum_chain(rows, dst, atoms, node_scale)
            out[f"segment_sum_C{channels}"] = {"eager_ms": round(median_eager(call), 4),
                                               "kernel_ms": round(time_steps(call, 1, steps, 10), 4),
                                               "torch_gpu_ms": round(median_eager(chain), 4),
                                               "dcu_ms": None, "source": "not published by the reference"}
        # tests/csrc/latency/test_rmsnorm_latency.py: 20 warmup calls, 7 repeats of 100 calls between
        # events, median and p95 of the per-call time, scale of ones; no figure is published
        for rows, width in ((1, 128), (32, 256), (128, 512), (512, 1024)):
            x = torch.randn(rows, width, generator=generator, device="cuda")
            scale = torch.ones(width, device="cuda")
            call = lambda _=None, x=x, scale=scale: kernels.rmsnorm(x, scale)
            for _ in range(20):
                call()
            torch.cuda.synchronize()
            samples = []
            for _ in range(7):
                start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                start.record()
                for _ in range(100):
                    call()
                stop.record()
                stop.synchronize()
                samples.append(start.elapsed_time(stop) / 100 * 1e3)
            samples.sort()
            out[f"rmsnorm_{rows}x{width}"] = {
                "eager_median_us": round(samples[3], 2), "eager_p95_us": round(samples[min(6, int(0.95 * 7))], 2),
                "kernel_us": round(time_steps(call, 1, steps, 10) * 1e3, 2),
                "dcu_ms": None, "source": "tests/csrc/latency/test_rmsnorm_latency.py (no figure published)"}
    out["note"] = ("same inputs every call, as in the reference's harness, so they stay in the Infinity Cache; "
                   "eager times include the Python layer's cost per call")
    return out


def op_line(name: str, job: dict, unit_count: int, unit: str = "edges/s") -> dict:
    line = {"op": name, "value": round(unit_count / (job["ms_per_step"] * 1e-3), 1), "unit": unit,
            "ms_per_step": round(job["ms_per_step"], 5), "input_sets": job.get("sets", 1),
            "roofline": roofline(job["bytes"], job["ms_per_step"])}
    for key in ("edges", "nodes", "channels", "rows", "width", "dtype"):
        if key in job:
            line[key] = job[key]
    return line


# ---------------------------------------------------------------------------
# CPU baselines (the oracle on the host cores)
# ---------------------------------------------------------------------------

def cpu_model() -> str:
    """The host CPU's model name (lscpu's "Model name"), read from /proc/cpuinfo."""
    try:
        with open("/proc/cpuinfo") as info:
            for row in info:
                if row.startswith("model name"):
                    return row.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baselines(softmax_case, seconds: float, extra_ops: dict | None) -> tuple[dict, dict]:
    import torch

    from oracle import segment as ref

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    c = {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in softmax_case.items()}

    def oracle():
        return ref.segment_softmax_reference(c["logit"], c["env"], c["dst"], c["offsets"], c["null_logit"])

    per_call, samples = cpu_time(oracle, seconds)
    edges = int(c["logit"].shape[0])
    headline = {"value": round(edges / per_call, 1), "unit": "edges/s", "cores": threads, "kind": "port",
                "sample": f"config 2 full input (E={edges}, C=8, null logit); median of {samples} calls of the "
                          f"oracle ATen chain (torch CPU, {threads} threads)",
                "ms_per_call": round(per_call * 1e3, 3), "cpu_model": cpu_model()}
    # the same chain on one core
    torch.set_num_threads(1)
    try:
        per_one, samples_one = cpu_time(oracle, min(seconds, 6.0))
    finally:
        torch.set_num_threads(threads)
    headline["single_thread"] = {"value": round(edges / per_one, 1), "ms_per_call": round(per_one * 1e3, 3),
                                 "calls": samples_one}
    extras = {}
    if extra_ops:
        for name, (function, count, description) in extra_ops.items():
            per, n = cpu_time(function, min(seconds, 5.0))
            extras[name] = {"value": round(count / per, 1), "unit": "edges/s", "sample": description,
                            "cores": threads, "ms_per_call": round(per * 1e3, 3), "calls": n}
    return headline, extras


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported in this build "
              "(the operators shard by destination-node ranges; see DESIGN.md)", file=sys.stderr)
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a gfx950 GPU", file=sys.stderr)
        return 1
    torch.cuda.set_device(0)
    from bysj_amd import kernels

    if not kernels.segment_available():
        print("libdpa4k.so is not usable on this device (build it with __graft_entry__.build())", file=sys.stderr)
        return 1
    graph = not args.eager
    print(f"[bench] headline: segment_softmax config 2, {args.steps} steps, {args.warmup} warmup", file=sys.stderr,
          flush=True)
    head = softmax_job(16384, args.steps, args.warmup, graph)
    value = head["edges"] / (head["ms_per_step"] * 1e-3)
    line = {
        "metric": "segment-op edges/s + % HBM roofline (segment_softmax forward, config 2)",
        "value": round(value, 1),
        "unit": "edges/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded; BASELINE.json config 2 generator)",
        "config": {"workload": "segment_softmax_fwd_config2", "nodes": head["nodes"], "edges": head["edges"],
                   "channels": head["channels"], "hub_fraction": 0.01, "hub_degree": 512, "null_logit": True,
                   "input_sets": head["sets"], "timing": "hip-graph replay" if graph else "eager",
                   "parallelism": "single-gpu"},
        "roofline": roofline(head["bytes"], head["ms_per_step"], "segment_softmax_fwd_config2"),
    }
    print(f"[bench] headline done: {head['ms_per_step'] * 1e3:.2f} us/step", file=sys.stderr, flush=True)
    edges, channels, nodes = head["edges"], head["channels"], head["nodes"]
    head_reads = edges * channels * 4 + edges * 4 + (nodes + 1) * 8 + nodes * channels * 4
    ceilings = stream_ceilings(head_reads, head["bytes"] - head_reads, args.steps)
    ceilings["headline_share_of_same_bytes_copy"] = round(ceilings["same_bytes_copy_us"] /
                                                          (head["ms_per_step"] * 1e3), 4)
    line["stream_ceilings"] = ceilings
    print("[bench] stream ceilings done", file=sys.stderr, flush=True)

    ops = {}
    extra_cpu = {}
    if not args.headline_only:
        from oracle import gie as gie_ref
        from oracle import segment as ref

        steps = max(10, args.steps // 4)
        warm = max(2, args.warmup // 4)
        job = segment_sum_job(1024, steps, warm, graph)
        ops["segment_sum_config1"] = op_line("segment_sum_fwd", job, job["edges"])
        b = {k: (v.cpu() if v is not None else None) for k, v in job["base"].items()}
        extra_cpu["segment_sum_config1"] = (
            lambda b=b: ref.segment_sum_reference(b["src"], b["dst"], b["offsets"]), job["edges"],
            "config 1 full input, oracle zeros->index_add_ chain")
        print("[bench] segment_sum config 1 done", file=sys.stderr, flush=True)
        gie, rms, water3, case3 = gie_rmsnorm_jobs(24576, steps, warm, graph)
        ops["gie_config3"] = op_line("gie_zonal_scatter_fwd", gie, gie["edges"])
        ops["rmsnorm_config3"] = op_line("rmsnorm_fwd", rms, rms["rows"], unit="rows/s")
        ops["gie_rmsnorm_config3"] = op_line("gie_zonal_scatter_rmsnorm_fwd", gie["fused_rmsnorm"], gie["edges"])
        ops["gie_rmsnorm_config3"]["unfused_ms_per_step"] = round(gie["ms_per_step"] + rms["ms_per_step"], 5)
        sample_nodes = 2048
        cut = int(water3.offsets()[sample_nodes])
        sample = tuple(t.cpu() for t in (case3["zonal"][:cut], case3["radial"][:cut], case3["dst"][:cut],
                                         case3["radial_slot"], case3["inv_sqrt_deg"][:sample_nodes]))
        extra_cpu["gie_config3"] = (lambda s=sample: gie_ref.zonal_scatter_reference(*s), cut,
                                    f"first {sample_nodes} atoms of config 3 ({cut} edges), oracle chain")
        del case3
        print("[bench] gie + rmsnorm config 3 done", file=sys.stderr, flush=True)
        from bysj_amd import workloads

        water4 = workloads.water_graph(65536, seed=0)
        for dtype_name in ("f32", "f64"):
            job, _, base = force_job(65536, steps, warm, graph, dtype_name, water=water4)
            ops[f"force_assembly_config4_{dtype_name}"] = op_line("force_assembly", job, job["edges"])
            bb = {k: v.cpu() for k, v in base.items()}
            extra_cpu[f"force_assembly_config4_{dtype_name}"] = (
                lambda bb=bb: ref.force_assembly_reference(bb["grad_edge"], bb["edge_vec"], bb["src"], bb["dst"],
                                                           bb["dst_offsets"], bb["src_offsets"]),
                job["edges"], f"config 4 full input ({dtype_name}), oracle two index_add_ + outer product")
            print(f"[bench] force config 4 {dtype_name} done", file=sys.stderr, flush=True)
        # the same box with atoms numbered in spatial (Morton) order, as MD engines sort them
        water4s = workloads.water_graph(65536, seed=0, spatial_order=True)
        for dtype_name in ("f32", "f64"):
            job, _, _ = force_job(65536, steps, warm, graph, dtype_name, water=water4s)
            ops[f"force_assembly_config4_{dtype_name}_spatial"] = op_line("force_assembly", job, job["edges"])
        print("[bench] force config 4 spatial order done", file=sys.stderr, flush=True)
        if not args.no_backward:
            job = softmax_backward_job(16384, steps, warm, graph)
            ops["segment_softmax_bwd_config2"] = op_line("segment_softmax_bwd", job, job["edges"])
            job = segment_sum_backward_job(1024, steps, warm, graph)
            ops["segment_sum_bwd_config1"] = op_line("segment_sum_bwd", job, job["edges"])
            job = segment_sum_backward_job(262144, max(4, steps // 4), warm, graph)
            ops["segment_sum_bwd_config1R"] = op_line("segment_sum_bwd", job, job["edges"])
            case3 = workloads.gie_config(water3, seed=0, device="cuda", primary=True)
            gie_b, rms_b = gie_rmsnorm_backward_jobs(water3, case3, steps, warm, graph)
            del case3
            ops["gie_bwd_config3"] = op_line("gie_zonal_scatter_bwd", gie_b, gie_b["edges"])
            ops["rmsnorm_bwd_config3"] = op_line("rmsnorm_bwd", rms_b, rms_b["rows"], unit="rows/s")
            job = csr_job(water4, steps, warm, graph)
            line_csr = op_line("group_by_source", job, job["edges"])
            line_csr["eager_ms_per_call"] = round(job["eager_ms_per_call"], 5)
            line_csr["torch_argsort_bincount_ms"] = round(job["torch_ms_per_call"], 5)
            ops["group_by_source_config4"] = line_csr
            print("[bench] backward kernels and CSR build done", file=sys.stderr, flush=True)
        if args.roofline_shapes:
            job = segment_sum_job(262144, steps, warm, graph)
            ops["segment_sum_config1R"] = op_line("segment_sum_fwd", job, job["edges"])
            job = segment_sum_job(262144, steps, warm, graph, scaled_shuffled=True)
            ops["segment_sum_config1R_scaled_shuffled"] = op_line("segment_sum_fwd", job, job["edges"])
            job = softmax_job(210000, steps, warm, graph)
            ops["segment_softmax_config2R"] = op_line("segment_softmax_fwd", job, job["edges"])
            if not args.no_backward:
                job = softmax_backward_job(210000, steps, warm, graph)
                ops["segment_softmax_bwd_config2R"] = op_line("segment_softmax_bwd", job, job["edges"])
            print("[bench] roofline shapes 1R, 2R done", file=sys.stderr, flush=True)
            water4r = workloads.water_graph(131072, seed=0)
            for dtype_name in ("f32", "f64"):
                job, _, _ = force_job(131072, steps, warm, graph, dtype_name, water=water4r)
                ops[f"force_assembly_config4R_{dtype_name}"] = op_line("force_assembly", job, job["edges"])
            del water4r
            print("[bench] roofline shape 4R done", file=sys.stderr, flush=True)
            # config 3R: 114,688 atoms (E ~ 10.4M; GIE radial [E, 16, 64] is 42.6 GB), two GIE steps
            water3r = workloads.water_graph(114688, seed=0)
            gie, rms, _, case3r = gie_rmsnorm_jobs(114688, steps, warm, graph, water=water3r, gie_steps=2)
            ops["gie_config3R"] = op_line("gie_zonal_scatter_fwd", gie, gie["edges"])
            ops["rmsnorm_config3R"] = op_line("rmsnorm_fwd", rms, rms["rows"], unit="rows/s")
            ops["gie_rmsnorm_config3R"] = op_line("gie_zonal_scatter_rmsnorm_fwd", gie["fused_rmsnorm"],
                                                  gie["edges"])
            ops["gie_rmsnorm_config3R"]["unfused_ms_per_step"] = round(gie["ms_per_step"] + rms["ms_per_step"], 5)
            if not args.no_backward:
                gie_b, rms_b = gie_rmsnorm_backward_jobs(water3r, case3r, steps, warm, graph, gie_steps=2)
                ops["gie_bwd_config3R"] = op_line("gie_zonal_scatter_bwd", gie_b, gie_b["edges"])
                ops["rmsnorm_bwd_config3R"] = op_line("rmsnorm_bwd", rms_b, rms_b["rows"], unit="rows/s")
            del case3r, water3r
            torch.cuda.empty_cache()
            print("[bench] roofline shape 3R done", file=sys.stderr, flush=True)
            rms, rms_b = rmsnorm_jobs(1048576, steps, warm, graph)
            ops["rmsnorm_rows1M"] = op_line("rmsnorm_fwd", rms, rms["rows"], unit="rows/s")
            ops["rmsnorm_bwd_rows1M"] = op_line("rmsnorm_bwd", rms_b, rms_b["rows"], unit="rows/s")
            print("[bench] roofline shapes done", file=sys.stderr, flush=True)
        for key, op in ops.items():
            op["roofline"]["traffic"] = measured_traffic(key, op["roofline"]["algorithmic_bytes"])
        line["ops"] = ops
        line["reference_shapes"] = reference_shapes(steps)
        print("[bench] reference latency shapes done", file=sys.stderr, flush=True)

    # BASELINE.json config 5 (DPA4Model(fused=True) end to end at 32,768 atoms) needs a DPA4/SeZM
    # model created by DeepMD-kit and DeepMD's own DeepPot; without DeepMD there is nothing to run.
    import importlib.util

    if importlib.util.find_spec("deepmd") is None:
        line["config5_dpa4_end_to_end"] = {
            "status": "unavailable", "unit": "atom-steps/s", "value": None,
            "reason": "deepmd-kit is not importable on this box and cannot be installed offline; the seam "
                      "layer (bysj_amd/model) is tested against stand-ins of DeepMD's seam functions instead"}
    else:
        line["config5_dpa4_end_to_end"] = {
            "status": "not run", "unit": "atom-steps/s", "value": None,
            "reason": "deepmd-kit is importable, but no frozen DPA4 model is available to this benchmark"}

    if args.calibrate_copy:
        source = torch.ones(64 * 2**20, dtype=torch.float32, device="cuda")
        target = torch.empty_like(source)
        target.copy_(source)
        torch.cuda.synchronize()
        line["calibration_copy_bytes"] = {"read": source.numel() * 4, "write": target.numel() * 4}

    if not args.no_cpu_baseline:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        headline_cpu, extras = cpu_baselines(head["base"], args.cpu_seconds, extra_cpu)
        line["cpu_baseline"] = headline_cpu
        for name, result in extras.items():
            if name in ops:
                ops[name]["cpu_baseline"] = result
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
