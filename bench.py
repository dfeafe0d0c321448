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
repeats the measurement for the other operators at their configuration sizes
and at the >=10M-edge roofline shapes (1R, 2R, 3R, 4R and 1M RMSNorm rows);
each large line also carries a same-run plain copy of its own read and write
bytes (`same_bytes_copy_us`) and its share of that copy.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--headline-only] [--no-roofline-shapes]
       python bench.py --traffic-summary FETCH_CSV WRITE_CSV BENCH_LOG   (see PMC_COMMAND)
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
    parser.add_argument("--no-roofline-shapes", action="store_true",
                        help="skip the >=10M-edge shapes (1R, 2R, 3R, 4R, 1M RMSNorm rows)")
    parser.add_argument("--traffic-marks", action="store_true",
                        help="eager launches with marker kernels around every step and a 256 MiB calibration "
                             "copy, for two rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE)")
    parser.add_argument("--only-force", choices=("f32", "f64"),
                        help="run only force_assembly on config 4 (random numbering) in this dtype, for a counter "
                             "profile of its kernels (FORCE_COUNTER_COMMANDS), and print one JSON line")
    parser.add_argument("--counter-table", nargs="+", metavar="COUNTER_CSV",
                        help="print, per kernel, the median per dispatch of every counter in rocprofv3 --pmc "
                             "counter CSVs (one pass each) as a Markdown table, then exit")
    parser.add_argument("--trace-summary", nargs=3, metavar=("STATS_CSV", "TRACE_CSV", "BENCH_LOG"),
                        help="write profiles/all_ops_kernel_stats.md from a rocprofv3 kernel trace of the default "
                             "bench (TRACE_COMMAND), then exit")
    parser.add_argument("--traffic-summary", nargs=3, metavar=("FETCH_CSV", "WRITE_CSV", "BENCH_LOG"),
                        help="write profiles/traffic.json and traffic.md from the two passes' counter CSVs and "
                             "the FETCH pass's bench output, then exit")
    return parser.parse_args()


# ---------------------------------------------------------------------------
# timing harness
# ---------------------------------------------------------------------------

class TrafficMarks:
    """Marker launches that split a rocprofv3 --pmc dispatch list into bench lines and steps.

    A marker is dpa4k_stream_calibrate's read-only kernel over `blocks` x 4096 floats, which
    runs exactly `blocks` workgroups: 1 opens a step, 2 closes a line, 3 + k opens line k of
    `labels`.  Every other launch of that kernel here reads 1 GiB (8,192 workgroups), so a
    launch of fewer than 256 workgroups is a marker.  traffic_summary() reads them back.
    """

    STEP, END, FIRST_LABEL = 1, 2, 3

    def __init__(self):
        import torch

        from bysj_amd.kernels import _lib

        self.labels: list[str] = []
        self._library = _lib.load()
        self._source = torch.zeros(4096 * 255, device="cuda")
        self._sink = torch.zeros(256, device="cuda")

    def _launch(self, blocks: int) -> None:
        import torch

        from bysj_amd.kernels import _lib

        _lib.check(self._library.dpa4k_stream_calibrate(self._source.data_ptr(), 4096 * blocks, self._sink.data_ptr(),
                                                        0, torch.cuda.current_stream().cuda_stream))

    def begin(self, label: str) -> None:
        if label in self.labels or len(self.labels) + self.FIRST_LABEL > 255:
            raise ValueError(f"traffic mark {label!r} repeated or past the marker range")
        self.labels.append(label)
        self._launch(self.FIRST_LABEL + len(self.labels) - 1)

    def step(self) -> None:
        self._launch(self.STEP)

    def end(self) -> None:
        self._launch(self.END)


MARKS: TrafficMarks | None = None  # set by --traffic-marks


def time_steps(step, n_sets: int, steps: int, warmup: int, *, graph: bool = True, label: str | None = None) -> float:
    """Average milliseconds per step over `steps` steps (step(i) uses input set i % n_sets).

    With --traffic-marks and a `label`, every step is launched eagerly behind a step marker,
    inside a begin/end pair for the label, so that a counter pass can price each step.
    """
    import torch

    marks = MARKS if label is not None else None
    if marks is not None:
        graph = False
        marks.begin(label)
    for i in range(warmup):
        if marks is not None:
            marks.step()
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
        # one untimed replay first: a graph's first launch also uploads it (about 7-10 us for the
        # headline's 20-step graph, 0.3-0.5 us a step); the timed replay then runs the same K steps
        hip_graph.replay()
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
            if marks is not None:
                marks.step()
            step(i % n_sets)
        stop.record(stream)
        torch.cuda.synchronize()
        elapsed = start.elapsed_time(stop)
    if marks is not None:
        marks.end()
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

def softmax_job(n_nodes: int, steps: int, warmup: int, graph: bool, label: str | None = None):
    import torch

    from bysj_amd import kernels, workloads

    base = workloads.segment_softmax_config(n_nodes=n_nodes, seed=0, device="cuda")
    edges, channels = base["logit"].shape
    offsets = base["offsets"]
    reads = edges * channels * 4 + edges * 4 + (n_nodes + 1) * 8 + n_nodes * channels * 4
    bytes_per_step = reads + edges * channels * 4 + n_nodes * channels * 4
    n_sets = n_sets_for(bytes_per_step)
    # one graph; every input set draws fresh logits, envelopes and null logits
    sets = [base] + [workloads.segment_softmax_features(edges, n_nodes, channels, seed=s, device="cuda")
                     for s in range(1, n_sets)]

    def step(i):
        case = sets[i]
        return kernels.segment_softmax(case["logit"], case["env"], offsets, case["null_logit"])

    with torch.no_grad():
        ms = time_steps(step, n_sets, steps, warmup, graph=graph, label=label)
    return {"edges": int(edges), "nodes": n_nodes, "channels": int(channels), "sets": n_sets,
            "ms_per_step": ms, "bytes": bytes_per_step, "reads": reads, "base": base}


def segment_sum_job(n_nodes: int, steps: int, warmup: int, graph: bool, scaled_shuffled: bool = False,
                    label: str | None = None):
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
        ms = time_steps(step, n_sets, steps, warmup, graph=graph, label=label)
    return {"edges": int(edges), "nodes": n_nodes, "channels": int(channels), "sets": n_sets,
            "ms_per_step": ms, "bytes": bytes_per_step, "reads": bytes_per_step - n_nodes * channels * 4,
            "base": base}


def gie_bytes(case, n_atoms: int, backward: bool = False) -> tuple[int, int]:
    """(reads, writes) of one GIE zonal-scatter launch over a destination CSR.

    Forward: zonal, every referenced radial slot, offsets, the slot map and the inverse degrees
    read once; the [N, R + 1, C] output written once.  Backward: the upstream gradient's rows
    1..R, zonal, the referenced radial slots, offsets, slot map and inverse degrees read; the
    zonal, radial (every slot: unreferenced ones are written as zeros) and inverse-degree
    gradients written.
    """
    edges, rows = case["zonal"].shape
    slots, channels = case["radial"].shape[1:]
    referenced = len(set(case["radial_slot"].tolist()))
    index = (n_atoms + 1) * 8 + rows * 8 + n_atoms * 4
    if not backward:
        return edges * rows * 4 + edges * referenced * channels * 4 + index, n_atoms * (rows + 1) * channels * 4
    reads = n_atoms * rows * channels * 4 + edges * rows * 4 + edges * referenced * channels * 4 + index
    return reads, edges * rows * 4 + edges * slots * channels * 4 + n_atoms * 4


def gie_forward_jobs(water, case, steps: int, warmup: int, graph: bool, gie_steps=None,
                     labels: tuple = (None, None, None)):
    """GIE forward, the fused GIE -> RMSNorm forward and RMSNorm forward on a water box.

    `labels` names the three lines (GIE, fused, RMSNorm); a None label skips that line.  GIE
    inputs are large enough (>= 1.7 GB of radial features at config 3) to stream from HBM with
    one input set; RMSNorm rotates through fresh rows.
    """
    import torch

    from bysj_amd.kernels import _C

    n_atoms = water.n_atoms
    gie_label, fused_label, rms_label = labels
    offsets, order, info = _C.gie_group(case["dst"], case["radial_slot"], n_atoms, case["radial"].shape[1])
    reads, writes = gie_bytes(case, n_atoms)
    rows = case["zonal"].shape[1]
    width = (rows + 1) * case["radial"].shape[2]
    count = gie_steps or max(4, steps // 10)
    out = {}
    with torch.no_grad():
        def gie_step(_):
            return _C.gie_zonal_scatter_forward_csr(case["zonal"], case["radial"], offsets, order,
                                                    case["radial_slot"], case["inv_sqrt_deg"], info)

        def fused_step(_):
            return _C.gie_rmsnorm_forward_csr(case["zonal"], case["radial"], offsets, order, case["radial_slot"],
                                              case["inv_sqrt_deg"], case["rms_scale"], 1e-6, False)

        if gie_label is not None:
            ms = time_steps(gie_step, 1, count, min(warmup, 3), graph=graph, label=gie_label)
            out["gie"] = {"edges": water.n_edges, "nodes": n_atoms, "ms_per_step": ms, "bytes": reads + writes,
                          "reads": reads, "sets": 1}
        if fused_label is not None:
            # the output is written once, normalised; scale and inverse RMS are the extra bytes
            fused_reads, fused_writes = reads + width * 4, writes + n_atoms * 4
            ms = time_steps(fused_step, 1, count, min(warmup, 3), graph=graph, label=fused_label)
            out["fused"] = {"edges": water.n_edges, "nodes": n_atoms, "ms_per_step": ms,
                            "bytes": fused_reads + fused_writes, "reads": fused_reads, "sets": 1}
        if rms_label is not None:
            x = gie_step(0).reshape(n_atoms, width)
            rms_reads = n_atoms * width * 4 + width * 4
            rms_bytes = rms_reads + n_atoms * width * 4 + n_atoms * 4
            n_sets = n_sets_for(rms_bytes)
            generator = torch.Generator(device="cuda")
            generator.manual_seed(3)
            row_sets = [x] + [torch.randn(x.shape, generator=generator, device="cuda") for _ in range(1, n_sets)]
            ms = time_steps(lambda i: _C.rmsnorm_forward(row_sets[i], case["rms_scale"], 1e-6), n_sets, steps,
                            warmup, graph=graph, label=rms_label)
            out["rms"] = {"rows": n_atoms, "width": width, "ms_per_step": ms, "bytes": rms_bytes,
                          "reads": rms_reads, "sets": n_sets}
    return out


def force_job(n_atoms: int, steps: int, warmup: int, graph: bool, dtype_name: str, water=None, label=None):
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
        ms = time_steps(step, n_sets, steps, warmup, graph=graph, label=label)
    return {"edges": edges, "nodes": n_atoms, "ms_per_step": ms, "bytes": bytes_per_step, "sets": n_sets,
            "reads": bytes_per_step - n_atoms * 12 * size,
            "dtype": dtype_name}, water, base


def softmax_backward_job(n_nodes: int, steps: int, warmup: int, graph: bool, label=None):
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

    ms = time_steps(step, n_sets, steps, warmup, graph=graph, label=label)
    return {"edges": int(edges), "nodes": n_nodes, "channels": int(channels), "sets": n_sets, "ms_per_step": ms,
            "bytes": reads + writes, "reads": reads}


def segment_sum_backward_job(n_nodes: int, steps: int, warmup: int, graph: bool, label=None):
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

    ms = time_steps(step, n_sets, steps, warmup, graph=graph, label=label)
    return {"edges": int(edges), "nodes": n_nodes, "channels": int(channels), "sets": n_sets, "ms_per_step": ms,
            "bytes": reads + writes, "reads": reads}


def gie_backward_job(water, case, steps: int, warmup: int, graph: bool, gie_steps=None, label=None):
    """GIE backward (zonal, radial and inverse-degree gradients) on a water box, one input set."""
    import torch

    from bysj_amd.kernels import _C

    n_atoms = water.n_atoms
    rows, channels = case["zonal"].shape[1], case["radial"].shape[2]
    offsets, order, info = _C.gie_group(case["dst"], case["radial_slot"], n_atoms, case["radial"].shape[1])
    generator = torch.Generator(device="cuda")
    generator.manual_seed(9)
    grad_out = torch.randn((n_atoms, rows + 1, channels), generator=generator, device="cuda")

    def step(_):
        return _C.gie_zonal_scatter_backward_csr(grad_out, case["zonal"], case["radial"], offsets, order,
                                                 case["radial_slot"], case["inv_sqrt_deg"], info)

    reads, writes = gie_bytes(case, n_atoms, backward=True)
    ms = time_steps(step, 1, gie_steps or max(4, steps // 10), min(warmup, 3), graph=graph, label=label)
    return {"edges": water.n_edges, "nodes": n_atoms, "ms_per_step": ms, "bytes": reads + writes, "reads": reads,
            "sets": 1, "shared_slots": not bool(info & 2)}


def rmsnorm_jobs(rows: int, steps: int, warmup: int, graph: bool, labels: tuple = (None, None)):
    """RMSNorm forward and backward over `rows` random rows of width 1024 (eps 1e-6, scale ~U(0.5, 1.5)).

    `labels` names the forward and backward lines; a None label skips that line.
    """
    import torch

    from bysj_amd.kernels import _C

    fwd_label, bwd_label = labels
    generator = torch.Generator(device="cuda")
    generator.manual_seed(13)
    scale = torch.rand(1024, generator=generator, device="cuda") + 0.5
    fwd_reads = rows * 1024 * 4 + 1024 * 4
    fwd_bytes = fwd_reads + rows * 1024 * 4 + rows * 4
    bwd_reads = 2 * rows * 1024 * 4 + 1024 * 4 + rows * 4
    bwd_bytes = bwd_reads + rows * 1024 * 4 + 1024 * 4
    n_sets = n_sets_for(bwd_bytes)
    sets = []
    for _ in range(n_sets):
        x = torch.randn((rows, 1024), generator=generator, device="cuda")
        _, inverse_rms = _C.rmsnorm_forward(x, scale, 1e-6)
        sets.append((x, inverse_rms, torch.randn((rows, 1024), generator=generator, device="cuda")))
    out = {}
    if fwd_label is not None:
        with torch.no_grad():
            ms = time_steps(lambda i: _C.rmsnorm_forward(sets[i][0], scale, 1e-6), n_sets, steps, warmup,
                            graph=graph, label=fwd_label)
        out["fwd"] = {"rows": rows, "width": 1024, "ms_per_step": ms, "bytes": fwd_bytes, "reads": fwd_reads,
                      "sets": n_sets}
    if bwd_label is not None:
        ms = time_steps(lambda i: _C.rmsnorm_backward(sets[i][2], sets[i][0], scale, sets[i][1], True), n_sets,
                        steps, warmup, graph=graph, label=bwd_label)
        out["bwd"] = {"rows": rows, "width": 1024, "ms_per_step": ms, "bytes": bwd_bytes, "reads": bwd_reads,
                      "sets": n_sets}
    return out


def edge_stream_job(n_edges: int, steps: int, warmup: int, graph: bool, label=None):
    """Fused edge-stream chain over [E, 10, 64]: out = silu(x + a * s + b), s one value per (edge, row).

    The shape and the chain are the reference's typical elementwise triple over [1, E, 10, 64]
    (docs/task2-hip-fusion-plan.md:282-284: residual add, per-row gate, accumulate) with the
    activation its design adds (:289).  `torch_chain_ms` times the eager chain the fused kernel
    replaces (t = a * s; t += x; t += b; silu(t): four passes, ten [E, 10, 64] streams against the
    fused kernel's four) on the same tensors.  One input set: each of the three inputs is larger
    than the Infinity Cache.
    """
    import torch

    from bysj_amd.kernels import _C

    shape = (n_edges, 10, 64)
    generator = torch.Generator(device="cuda")
    generator.manual_seed(23)
    x, a, b = (torch.randn(shape, generator=generator, device="cuda") for _ in range(3))
    s = torch.randn((n_edges, 10, 1), generator=generator, device="cuda")
    out = torch.empty(shape, device="cuda")
    full = n_edges * 640 * 4
    reads = 3 * full + n_edges * 10 * 4
    terms = [(1.0, x, None), (1.0, a, s), (1.0, b, None)]

    def chain(_):
        # nothing is returned, so a captured step's [E, 10, 64] temporary goes back to the
        # graph's pool for the next step (kept outputs would hold one per step)
        t = a * s
        t += x
        t += b
        torch.nn.functional.silu(t, inplace=True)

    with torch.no_grad():
        ms = time_steps(lambda _: _C.edge_stream_combine(terms, shape, "silu", None, None, out), 1, steps, warmup,
                        graph=graph, label=label)
        torch_ms = time_steps(chain, 1, max(5, steps // 4), 2, graph=graph)
    del x, a, b, s, out, terms
    torch.cuda.empty_cache()
    return {"edges": n_edges, "rows": 10, "channels": 64, "ms_per_step": ms, "bytes": reads + full, "reads": reads,
            "sets": 1, "torch_chain_ms": torch_ms}


def csr_job(water, steps: int, warmup: int, graph: bool, label=None):
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
                    steps, warmup, graph=graph, label=label)
    statuses = [int(b["status"].item()) for b in buffers]
    if any(code & 1 for code in statuses):
        raise RuntimeError(f"group_by_key_async reported out-of-range keys: {statuses}")
    eager_ms = time_steps(lambda _: kernels.group_by_source(src, n_atoms), 1, max(5, steps // 4), 2, graph=False)
    torch_ms = time_steps(lambda _: (torch.argsort(src, stable=True),
                                     torch.bincount(src, minlength=n_atoms).cumsum(0)), 1, max(5, steps // 4), 2,
                          graph=False)
    return {"edges": edges, "nodes": n_atoms, "ms_per_step": ms, "bytes": bytes_per_step, "reads": edges * 8,
            "sets": n_sets, "eager_ms_per_call": eager_ms, "torch_ms_per_call": torch_ms}


def same_bytes_copy_ms(read_bytes: int, write_bytes: int, steps: int, warmup: int) -> tuple[float, int]:
    """Milliseconds per launch of a plain copy that reads `read_bytes` and writes `write_bytes`.

    The copy (dpa4k_stream_calibrate) streams through enough distinct sources to leave the
    Infinity Cache, like the operator lines, and is timed the same way.  Returns the time and
    the bytes the copy moved (the counts rounded up to whole 16-byte chunks; the writes are
    capped at the reads: every line priced this way reads at least as many bytes as it writes).
    """
    import torch

    from bysj_amd.kernels import _lib

    library = _lib.load()
    torch.cuda.empty_cache()
    read_floats = (read_bytes // 4 + 3) // 4 * 4
    write_floats = min(read_floats, (write_bytes // 4 + 3) // 4 * 4)
    n_sets = n_sets_for(read_bytes + write_bytes)
    sources = [torch.empty(read_floats, device="cuda") for _ in range(n_sets)]
    out = torch.empty(max(write_floats, 8192), device="cuda")

    def launch(i):
        _lib.check(library.dpa4k_stream_calibrate(sources[i].data_ptr(), read_floats, out.data_ptr(), write_floats,
                                                  torch.cuda.current_stream().cuda_stream))

    ms = time_steps(launch, n_sets, steps, warmup)
    del sources, out
    torch.cuda.empty_cache()
    return ms, (read_floats + write_floats) * 4


def copy_share(line: dict, job: dict, steps: int) -> dict:
    """Add the same-run copy of the line's own read and write bytes, and the line's share of it."""
    copy_ms, _ = same_bytes_copy_ms(job["reads"], job["bytes"] - job["reads"], steps, 3)
    line["same_bytes_copy_us"] = round(copy_ms * 1e3, 3)
    line["share_of_same_bytes_copy"] = round(copy_ms / job["ms_per_step"], 4)
    return line


def stream_ceilings(read_bytes: int, write_bytes: int, steps: int) -> dict:
    """Read-only and copy rates of plain streams on this part, and a copy of one operator's bytes.

    1 GiB read-only and copy passes (dpa4k_stream_calibrate: grid-stride, four 16-byte chunks per
    thread per round, non-temporal loads and stores), then a copy that reads `read_bytes` and writes `write_bytes`, rotated
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
    op_ms, moved = same_bytes_copy_ms(read_bytes, write_bytes, steps, 20)
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
    channels, segment_sum with a node scale at 64, 256 and 640 channels (its `_CHANNELS`, :49),
    force assembly on uniform random sources.  `eager_ms` follows its `_median_ms`
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
        for channels in (64, 256, 640):
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


# ---------------------------------------------------------------------------
# HBM traffic per step from two rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE)
# ---------------------------------------------------------------------------

PMC_COMMAND = ("timeout -s KILL 1100 rocprofv3 --pmc {counter} --output-format csv -d gpurun_out/pmc_{tag} -o run "
               "-- python3 -u bench.py --no-cpu-baseline --traffic-marks --steps 20 --warmup 5 "
               "> gpurun_out/pmc_{tag}.log 2>&1")
SUMMARY_COMMAND = ("python3 bench.py --traffic-summary gpurun_out/pmc_fetch/run_counter_collection.csv "
                   "gpurun_out/pmc_write/run_counter_collection.csv gpurun_out/pmc_fetch.log")
CALIBRATION_LABEL = "calibration_copy"
CALIBRATION_FLOATS = 64 * 2**20  # a 256 MiB read and a 256 MiB write


def _kernel_short(name: str) -> str:
    """A kernel's name without `void`, anonymous namespaces or the parameter list."""
    name = name.replace("(anonymous namespace)::", "")
    if name.startswith("void "):
        name = name[5:]
    depth = 0
    for i, ch in enumerate(name):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            return name[:i]
    return name


def _counter_dispatches(path: str, counter: str) -> list[tuple[str, int, float]]:
    """(kernel, workgroups, counter value in KiB) of every dispatch in a rocprofv3 --pmc CSV, in order."""
    import csv

    with open(path, newline="") as handle:
        rows = [row for row in csv.DictReader(handle) if row["Counter_Name"] == counter]
    rows.sort(key=lambda row: int(row["Dispatch_Id"]))
    return [(_kernel_short(row["Kernel_Name"]), int(row["Grid_Size"]) // max(1, int(row["Workgroup_Size"])),
             float(row["Counter_Value"])) for row in rows]


def _marked_steps(dispatches, labels: list[str]) -> dict:
    """{label: [[(kernel, workgroups, value), ...] for each step]} from TrafficMarks' markers."""
    lines, label, steps = {}, None, None
    for kernel, blocks, value in dispatches:
        if kernel.endswith("stream_read_kernel") and blocks < 256:
            if blocks >= TrafficMarks.FIRST_LABEL:
                label, steps = labels[blocks - TrafficMarks.FIRST_LABEL], []
            elif blocks == TrafficMarks.STEP and steps is not None:
                steps.append([])
            elif blocks == TrafficMarks.END and steps is not None:
                lines[label] = steps
                label, steps = None, None
            continue
        if steps:
            steps[-1].append((kernel, blocks, value))
    return lines


def _bench_json(path: str) -> dict:
    """The full bench line of a log: the ``detail`` line when the run printed one, else its last JSON line."""
    with open(path) as handle:
        rows = [json.loads(row) for row in handle if row.startswith("{")]
    if not rows:
        raise SystemExit(f"no bench JSON line in {path}")
    return next((row for row in rows if row.get("detail")), rows[-1])


def traffic_summary(fetch_csv: str, write_csv: str, bench_log: str, out_dir: Path | None = None) -> int:
    """Write profiles/traffic.json and profiles/traffic.md from one FETCH_SIZE and one WRITE_SIZE pass.

    Both passes run `bench.py --traffic-marks` under rocprofv3 --pmc (PMC_COMMAND).  Each bench
    line's steps are the dispatches between its step markers; a step's traffic is the sum over
    its dispatches of both counters, each scaled by what it reads for the calibration copy
    (256 MiB read, 256 MiB written by dpa4k_stream_calibrate).  The figure per line is the
    median over its steps after the first.
    """
    import statistics

    line = _bench_json(bench_log)
    labels = line.get("traffic_marks")
    if not labels:
        raise SystemExit(f"{bench_log} was not written by a --traffic-marks run")
    fetch = _marked_steps(_counter_dispatches(fetch_csv, "FETCH_SIZE"), labels)
    write = _marked_steps(_counter_dispatches(write_csv, "WRITE_SIZE"), labels)
    for label, steps in fetch.items():
        other = write.get(label)
        same = other is not None and [[d[:2] for d in st] for st in steps] == [[d[:2] for d in st] for st in other]
        if not same:
            raise SystemExit(f"the two passes launched different kernels for {label}")
    copy_bytes = CALIBRATION_FLOATS * 4
    fetch_scale = copy_bytes / (statistics.median(st[0][2] for st in fetch[CALIBRATION_LABEL]) * 1024)
    write_scale = copy_bytes / (statistics.median(st[0][2] for st in write[CALIBRATION_LABEL]) * 1024)
    algorithmic = {line["config"]["workload"]: line["roofline"]["algorithmic_bytes"]}
    algorithmic.update({key: op["roofline"]["algorithmic_bytes"] for key, op in line.get("ops", {}).items()})
    table, rows = {}, []
    for label in labels:
        if label == CALIBRATION_LABEL or label not in algorithmic or label not in fetch:
            continue
        steps_f, steps_w = fetch[label], write[label]
        counted = range(1, len(steps_f)) if len(steps_f) > 2 else range(len(steps_f))
        fetched = statistics.median(sum(d[2] for d in steps_f[i]) * 1024 * fetch_scale for i in counted)
        written = statistics.median(sum(d[2] for d in steps_w[i]) * 1024 * write_scale for i in counted)
        kernels = list(dict.fromkeys(d[0] for d in steps_f[counted[0]]))
        table[label] = {"bytes_per_launch": int(fetched + written), "fetch_bytes": int(fetched),
                        "write_bytes": int(written), "fetch_scale": round(fetch_scale, 4),
                        "write_scale": round(write_scale, 4), "algorithmic_bytes": int(algorithmic[label]),
                        "kernels": kernels, "steps": len(counted), "source": "profiles/traffic.md"}
        rows.append(f"| {label} | {', '.join(f'`{k}`' for k in kernels)} | {len(counted)} | {int(fetched):,} | "
                    f"{int(written):,} | {int(fetched + written):,} | {int(algorithmic[label]):,} | "
                    f"{(fetched + written) / algorithmic[label]:.3f} |")
    out = out_dir or ROOT / "profiles"
    (out / "traffic.json").write_text(json.dumps(table, indent=1) + "\n")
    calibration = statistics.median(st[0][2] for st in fetch[CALIBRATION_LABEL])
    text = [
        "# HBM traffic per step of every bench line (rocprofv3 FETCH_SIZE / WRITE_SIZE)", "",
        "Commands (repository root, one MI355X; one counter per pass, eager launches, each step "
        "bracketed by marker launches):", "", "```",
        PMC_COMMAND.format(counter="FETCH_SIZE", tag="fetch"),
        PMC_COMMAND.format(counter="WRITE_SIZE", tag="write"),
        SUMMARY_COMMAND, "```", "",
        f"Calibration: a plain copy of {copy_bytes:,} bytes (`dpa4k::stream_copy_kernel`) reads "
        f"{calibration:,.1f} KiB by FETCH_SIZE (scale {fetch_scale:.4f}) and writes "
        f"{copy_bytes / 1024 / write_scale:,.1f} KiB by WRITE_SIZE (scale {write_scale:.4f}).  Every figure below is "
        "scaled by these factors; a step's traffic is the sum over all of its dispatches (library and torch "
        "kernels alike), the median over its steps after the first.", "",
        "| Bench line | Kernels of a step | Steps | FETCH bytes | WRITE bytes | Traffic | Algorithmic bytes | "
        "Traffic / algorithmic |", "| --- | --- | --- | --- | --- | --- | --- | --- |", *rows, ""]
    (out / "traffic.md").write_text("\n".join(text))
    print(f"wrote {len(table)} lines to {out / 'traffic.json'} and traffic.md")
    return 0


FORCE_COUNTERS = (
    "SQ_WAVES SQ_WAVE_CYCLES SQ_BUSY_CYCLES SQ_INSTS_VALU SQ_INSTS_LDS SQ_LDS_BANK_CONFLICT SQ_INSTS_VMEM_RD "
    "SQ_INSTS_VMEM_WR GRBM_GUI_ACTIVE",
    "TCC_REQ_sum TCC_HIT_sum TCC_MISS_sum TCP_TCC_READ_REQ_sum TCP_TCC_READ_REQ_LATENCY_sum "
    "TCP_PENDING_STALL_CYCLES_sum TA_BUSY_avr GRBM_GUI_ACTIVE",
    "FETCH_SIZE",
    "WRITE_SIZE",
)
FORCE_COUNTER_COMMAND = ("timeout -s KILL 300 rocprofv3 --pmc {counters} --kernel-include-regex force_ "
                         "--output-format csv -d gpurun_out/pmc_force_{tag}_{dtype} -o run -- python3 bench.py "
                         "--only-force {dtype} --eager --steps 40 --warmup 4")


def counter_table(paths: list[str]) -> str:
    """Per kernel, the median per dispatch of every counter of one or more rocprofv3 --pmc CSVs."""
    import csv
    import statistics
    from collections import defaultdict

    values = defaultdict(lambda: defaultdict(list))
    for path in paths:
        with open(path, newline="") as handle:
            for row in csv.DictReader(handle):
                values[_kernel_short(row["Kernel_Name"])][row["Counter_Name"]].append(float(row["Counter_Value"]))
    names = sorted({counter for kernel in values.values() for counter in kernel})
    lines = ["| Kernel | Dispatches | " + " | ".join(names) + " |", "| --- | --- | " + " | ".join("---" for _ in names) + " |"]
    for kernel, counters in sorted(values.items()):
        dispatches = max(len(v) for v in counters.values())
        cells = [f"{statistics.median(counters[n]):,.0f}" if n in counters else "" for n in names]
        lines.append(f"| `{kernel}` | {dispatches} | " + " | ".join(cells) + " |")
    return "\n".join(lines)


TRACE_COMMAND = ("timeout -k 10 600 rocprofv3 --kernel-trace --stats --output-format csv -d gpurun_out/prof_ops -o run "
                 "-- python3 -u bench.py --no-cpu-baseline --steps 20 --warmup 5 > gpurun_out/prof_ops.log 2>&1")
TRACE_SUMMARY_COMMAND = ("python3 bench.py --trace-summary gpurun_out/prof_ops/run_kernel_stats.csv "
                         "gpurun_out/prof_ops/run_kernel_trace.csv gpurun_out/prof_ops.log")


def trace_summary(stats_csv: str, trace_csv: str, bench_log: str, out_dir: Path | None = None) -> int:
    """Write profiles/all_ops_kernel_stats.md from a rocprofv3 kernel trace of the default bench.

    Library kernels from the stats file (averaged over every shape the bench runs them at), the
    same trace by kernel and grid (median of a line's launches), and the bench's own per-step times
    of the same process beside them.
    """
    import csv
    import statistics
    from collections import defaultdict

    def short(name: str) -> str:
        return _kernel_short(name)

    rows = ["# Kernel durations of every bench line (rocprofv3 kernel trace)", "",
            "Commands (repository root, one MI355X):", "", "```", TRACE_COMMAND, TRACE_SUMMARY_COMMAND, "```", "",
            "Library kernels (`dpa4k::`) from `run_kernel_stats.csv`, averaged over every shape the bench runs for "
            "that kernel template (the calibration `stream_*` kernels measure the same-bytes copies and the stream "
            "ceilings):", "", "| Kernel | Calls | Average ns | Min ns | Max ns | % of GPU time |",
            "| --- | --- | --- | --- | --- | --- |"]
    with open(stats_csv, newline="") as handle:
        for r in csv.DictReader(handle):
            name = short(r["Name"])
            if name.startswith("dpa4k::"):
                rows.append(f"| `{name}` | {r['Calls']} | {float(r['AverageNs']):.0f} | {float(r['MinNs']):.0f} | "
                            f"{float(r['MaxNs']):.0f} | {float(r['Percentage']):.2f} |")
    groups = defaultdict(list)
    with open(trace_csv, newline="") as handle:
        for r in csv.DictReader(handle):
            name = short(r["Kernel_Name"])
            if not name.startswith("dpa4k::"):
                continue
            grid = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
            groups[(name, grid)].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0)
    rows += ["", "The same trace by kernel and grid (launches of at least 20, i.e. a line's warm-up and timed steps; "
             "median of the launches):", "", "| Kernel | Grid (work-items) | Launches | Median µs | Mean µs |",
             "| --- | --- | --- | --- | --- |"]
    for (name, grid), times in sorted(groups.items()):
        if len(times) >= 20:
            rows.append(f"| `{name}` | {grid:,} | {len(times)} | {statistics.median(times):.1f} | "
                        f"{statistics.mean(times):.1f} |")
    line = _bench_json(bench_log)
    rows += ["", "Bench `ms_per_step` of the same process (graph replay, HIP events), for comparison:", "",
             "| Bench line | µs per step | frac |", "| --- | --- | --- |",
             f"| {line['config']['workload']} (headline) | {line['ms_per_step'] * 1000:.2f} | "
             f"{line['roofline']['frac']} |"]
    for key, op in line.get("ops", {}).items():
        rows.append(f"| {key} | {op['ms_per_step'] * 1000:.2f} | {op['roofline']['frac']} |")
    out = (out_dir or ROOT / "profiles") / "all_ops_kernel_stats.md"
    out.write_text("\n".join(rows) + "\n")
    print(f"wrote {out}")
    return 0


# ---------------------------------------------------------------------------
# the final line
# ---------------------------------------------------------------------------

# one row per `ops` entry of the final line; the detail line carries every field
OPS_FIELDS = ("value", "unit", "us_per_step", "frac", "traffic_over_algorithmic", "share_of_same_bytes_copy",
              "achieved_GBps")
REFERENCE_FIELDS = ("eager_ms", "kernel_ms", "torch_gpu_ms", "dcu_ms", "dcu_torch_ms")
FINAL_LINE_LIMIT = 8000  # bytes: the driver keeps the last ~8.5 KB of the output


def _sig(value, digits: int = 4):
    """``value`` rounded to ``digits`` significant digits (None and strings unchanged)."""
    if not isinstance(value, (int, float)) or value == 0:
        return value
    return float(f"{value:.{digits}g}")


def compact_line(line: dict) -> dict:
    """The final JSON line: the headline's keys in full, every op as one row of OPS_FIELDS.

    The full line (every field of every op, the reference's latency shapes with their sources,
    the notes) is printed just before it with ``"detail": true``.
    """
    out = {key: value for key, value in line.items()
           if key not in ("ops", "reference_shapes", "config5_dpa4_end_to_end", "cpu_baseline", "stream_ceilings",
                          "traffic_marks")}
    if "stream_ceilings" in line:
        out["stream_ceilings"] = {k: v for k, v in line["stream_ceilings"].items() if k != "note"}
    if "cpu_baseline" in line:
        out["cpu_baseline"] = dict(line["cpu_baseline"])
    ops = line.get("ops", {})
    if ops:
        out["ops_fields"] = list(OPS_FIELDS)
        rows, cpu = {}, {}
        for key, op in ops.items():
            roof = op["roofline"]
            traffic = roof.get("traffic")
            ratio = round(traffic / roof["algorithmic_bytes"], 3) if traffic and roof["algorithmic_bytes"] else None
            rows[key] = [_sig(op["value"]), op["unit"], round(op["ms_per_step"] * 1e3, 2), roof["frac"], ratio,
                         op.get("share_of_same_bytes_copy"), round(roof["achieved"])]
            if "cpu_baseline" in op:
                c = op["cpu_baseline"]
                cpu[key] = [_sig(c["value"]), c["unit"], c["cores"]]
        out["ops"] = rows
        if cpu:
            out["ops_cpu_baseline_fields"] = ["value", "unit", "cores"]
            out["ops_cpu_baseline"] = cpu
    shapes = line.get("reference_shapes")
    if shapes:
        def ms(entry: dict, field: str):
            if field in entry:
                return entry[field]
            micro = {"eager_ms": "eager_median_us", "kernel_ms": "kernel_us"}.get(field)  # the RMSNorm rows
            return round(entry[micro] / 1e3, 5) if micro in entry else None

        out["reference_shapes_fields"] = list(REFERENCE_FIELDS)
        out["reference_shapes"] = {key: [ms(entry, field) for field in REFERENCE_FIELDS]
                                   for key, entry in shapes.items() if isinstance(entry, dict)}
    if "config5_dpa4_end_to_end" in line:
        c5 = line["config5_dpa4_end_to_end"]
        out["config5_dpa4_end_to_end"] = {"status": c5["status"], "unit": c5["unit"], "value": c5["value"]}
    text = json.dumps(out)
    if len(text) > FINAL_LINE_LIMIT:  # never expected: drop the secondary tables before the ops rows
        for key in ("reference_shapes", "reference_shapes_fields", "ops_cpu_baseline", "ops_cpu_baseline_fields"):
            out.pop(key, None)
    return out


# ---------------------------------------------------------------------------
# driver
# ---------------------------------------------------------------------------

def main() -> int:
    args = parse_args()
    if args.traffic_summary:
        return traffic_summary(*args.traffic_summary)
    if args.trace_summary:
        return trace_summary(*args.trace_summary)
    if args.counter_table:
        print(counter_table(args.counter_table))
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported in this build "
              "(the operators would shard by contiguous destination-node ranges, one range per GPU, "
              "with the ghost rows' partial sums exchanged; no multi-GPU path is built)", file=sys.stderr)
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
    graph = not (args.eager or args.traffic_marks)
    if args.only_force:
        job, _, _ = force_job(65536, args.steps, args.warmup, graph, args.only_force,
                              label=f"force_assembly_config4_{args.only_force}")
        print(json.dumps({"op": f"force_assembly_config4_{args.only_force}", "steps": args.steps,
                          "ms_per_step": round(job["ms_per_step"], 5), "edges": job["edges"],
                          "roofline": roofline(job["bytes"], job["ms_per_step"])}), flush=True)
        return 0
    global MARKS
    if args.traffic_marks:
        from bysj_amd.kernels import _lib

        MARKS = TrafficMarks()
        source = torch.zeros(CALIBRATION_FLOATS, device="cuda")
        target = torch.empty_like(source)
        library = _lib.load()
        time_steps(lambda _: _lib.check(library.dpa4k_stream_calibrate(
            source.data_ptr(), CALIBRATION_FLOATS, target.data_ptr(), CALIBRATION_FLOATS,
            torch.cuda.current_stream().cuda_stream)), 1, 3, 1, label=CALIBRATION_LABEL)
        del source, target

    def progress(what: str) -> None:
        print(f"[bench] {what}", file=sys.stderr, flush=True)

    progress(f"headline: segment_softmax config 2, {args.steps} steps, {args.warmup} warmup")
    head = softmax_job(16384, args.steps, args.warmup, graph, label="segment_softmax_fwd_config2")
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
    progress(f"headline done: {head['ms_per_step'] * 1e3:.2f} us/step")
    if not args.traffic_marks:
        ceilings = stream_ceilings(head["reads"], head["bytes"] - head["reads"], args.steps)
        ceilings["headline_share_of_same_bytes_copy"] = round(ceilings["same_bytes_copy_us"] /
                                                              (head["ms_per_step"] * 1e3), 4)
        line["stream_ceilings"] = ceilings
        progress("stream ceilings done")

    ops = {}
    extra_cpu = {}
    if not args.headline_only:
        from bysj_amd import workloads
        from oracle import gie as gie_ref
        from oracle import segment as ref

        steps = max(10, args.steps // 4)
        warm = max(2, args.warmup // 4)
        big = not args.no_roofline_shapes
        backward = not args.no_backward

        def add(key: str, name: str, job: dict, count: int, unit: str = "edges/s", share: bool = False) -> dict:
            entry = op_line(name, job, count, unit)
            if share and MARKS is None:
                copy_share(entry, job, steps)
            ops[key] = entry
            return entry

        # ---- segment_sum forward: config 1, 1R plain and 1R with scales and a shuffled order
        job = segment_sum_job(1024, steps, warm, graph, label="segment_sum_config1")
        add("segment_sum_config1", "segment_sum_fwd", job, job["edges"])
        b = {k: (v.cpu() if v is not None else None) for k, v in job["base"].items()}
        extra_cpu["segment_sum_config1"] = (
            lambda b=b: ref.segment_sum_reference(b["src"], b["dst"], b["offsets"]), job["edges"],
            "config 1 full input, oracle zeros->index_add_ chain")
        if big:
            job = segment_sum_job(262144, steps, warm, graph, label="segment_sum_config1R")
            add("segment_sum_config1R", "segment_sum_fwd", job, job["edges"], share=True)
            job = segment_sum_job(262144, steps, warm, graph, scaled_shuffled=True,
                                  label="segment_sum_config1R_scaled_shuffled")
            add("segment_sum_config1R_scaled_shuffled", "segment_sum_fwd", job, job["edges"], share=True)
            del job
            job = softmax_job(210000, steps, warm, graph, label="segment_softmax_config2R")
            add("segment_softmax_config2R", "segment_softmax_fwd", job, job["edges"], share=True)
            del job
        progress("segment_sum 1/1R and segment_softmax 2R forward done")

        # ---- GIE zonal scatter (primary [E,16,64] and DeepMD-shaped secondary [E,3,64]) -> RMSNorm, config 3
        water3 = workloads.water_graph(24576, seed=0)
        case3 = workloads.gie_config(water3, seed=0, device="cuda", primary=True)
        jobs = gie_forward_jobs(water3, case3, steps, warm, graph,
                                labels=("gie_config3", "gie_rmsnorm_config3", "rmsnorm_config3"))
        add("gie_config3", "gie_zonal_scatter_fwd", jobs["gie"], water3.n_edges, share=True)
        add("rmsnorm_config3", "rmsnorm_fwd", jobs["rms"], jobs["rms"]["rows"], unit="rows/s")
        fused = add("gie_rmsnorm_config3", "gie_zonal_scatter_rmsnorm_fwd", jobs["fused"], water3.n_edges)
        fused["unfused_ms_per_step"] = round(jobs["gie"]["ms_per_step"] + jobs["rms"]["ms_per_step"], 5)
        sample_nodes = 2048
        cut = int(water3.offsets()[sample_nodes])
        sample = tuple(t.cpu() for t in (case3["zonal"][:cut], case3["radial"][:cut], case3["dst"][:cut],
                                         case3["radial_slot"], case3["inv_sqrt_deg"][:sample_nodes]))
        extra_cpu["gie_config3"] = (lambda s=sample: gie_ref.zonal_scatter_reference(*s), cut,
                                    f"first {sample_nodes} atoms of config 3 ({cut} edges), oracle chain")
        if backward:
            job = gie_backward_job(water3, case3, steps, warm, graph, label="gie_bwd_config3")
            add("gie_bwd_config3", "gie_zonal_scatter_bwd", job, job["edges"], share=True)
        del case3
        case3s = workloads.gie_config(water3, seed=0, device="cuda", primary=False)
        jobs = gie_forward_jobs(water3, case3s, steps, warm, graph, labels=("gie_config3_secondary", None, None))
        add("gie_config3_secondary", "gie_zonal_scatter_fwd", jobs["gie"], water3.n_edges, share=True)
        sample = tuple(t.cpu() for t in (case3s["zonal"][:cut], case3s["radial"][:cut], case3s["dst"][:cut],
                                         case3s["radial_slot"], case3s["inv_sqrt_deg"][:sample_nodes]))
        extra_cpu["gie_config3_secondary"] = (lambda s=sample: gie_ref.zonal_scatter_reference(*s), cut,
                                              f"first {sample_nodes} atoms of config 3 secondary ({cut} edges), "
                                              "oracle chain")
        if backward:
            job = gie_backward_job(water3, case3s, steps, warm, graph, label="gie_bwd_config3_secondary")
            add("gie_bwd_config3_secondary", "gie_zonal_scatter_bwd", job, job["edges"], share=True)
            jobs = rmsnorm_jobs(24576, steps, warm, graph, labels=(None, "rmsnorm_bwd_config3"))
            add("rmsnorm_bwd_config3", "rmsnorm_bwd", jobs["bwd"], 24576, unit="rows/s")
        del case3s, sample
        torch.cuda.empty_cache()
        progress("gie + rmsnorm config 3 (primary, secondary) done")

        # ---- force assembly, config 4 (random and Morton atom numbering) and 4R
        water4 = workloads.water_graph(65536, seed=0)
        for dtype_name in ("f32", "f64"):
            key = f"force_assembly_config4_{dtype_name}"
            job, _, base = force_job(65536, steps, warm, graph, dtype_name, water=water4, label=key)
            add(key, "force_assembly", job, job["edges"])
            bb = {k: v.cpu() for k, v in base.items()}
            extra_cpu[key] = (
                lambda bb=bb: ref.force_assembly_reference(bb["grad_edge"], bb["edge_vec"], bb["src"], bb["dst"],
                                                           bb["dst_offsets"], bb["src_offsets"]),
                job["edges"], f"config 4 full input ({dtype_name}), oracle two index_add_ + outer product")
            del base
        # the same box with atoms numbered in spatial (Morton) order, as MD engines sort them
        water4s = workloads.water_graph(65536, seed=0, spatial_order=True)
        for dtype_name in ("f32", "f64"):
            key = f"force_assembly_config4_{dtype_name}_spatial"
            job, _, _ = force_job(65536, steps, warm, graph, dtype_name, water=water4s, label=key)
            add(key, "force_assembly", job, job["edges"])
        del water4s
        if big:
            water4r = workloads.water_graph(131072, seed=0)
            for dtype_name in ("f32", "f64"):
                key = f"force_assembly_config4R_{dtype_name}"
                job, _, _ = force_job(131072, steps, warm, graph, dtype_name, water=water4r, label=key)
                add(key, "force_assembly", job, job["edges"], share=True)
            del water4r
        torch.cuda.empty_cache()
        progress("force assembly config 4 / 4R done")

        # ---- backward kernels and the CSR build
        if backward:
            job = softmax_backward_job(16384, steps, warm, graph, label="segment_softmax_bwd_config2")
            add("segment_softmax_bwd_config2", "segment_softmax_bwd", job, job["edges"])
            job = segment_sum_backward_job(1024, steps, warm, graph, label="segment_sum_bwd_config1")
            add("segment_sum_bwd_config1", "segment_sum_bwd", job, job["edges"])
            if big:
                job = softmax_backward_job(210000, steps, warm, graph, label="segment_softmax_bwd_config2R")
                add("segment_softmax_bwd_config2R", "segment_softmax_bwd", job, job["edges"], share=True)
                job = segment_sum_backward_job(262144, max(4, steps // 4), warm, graph,
                                               label="segment_sum_bwd_config1R")
                add("segment_sum_bwd_config1R", "segment_sum_bwd", job, job["edges"], share=True)
            job = csr_job(water4, steps, warm, graph, label="group_by_source_config4")
            entry = add("group_by_source_config4", "group_by_source", job, job["edges"])
            entry["eager_ms_per_call"] = round(job["eager_ms_per_call"], 5)
            entry["torch_argsort_bincount_ms"] = round(job["torch_ms_per_call"], 5)
            torch.cuda.empty_cache()
            progress("backward kernels and CSR build done")
        del water4

        # ---- config 3R: 114,688 atoms (E ~ 10.4M; the primary radial [E, 16, 64] is 42.6 GB)
        if big:
            water3r = workloads.water_graph(114688, seed=0)
            case = workloads.gie_config(water3r, seed=0, device="cuda", primary=True)
            jobs = gie_forward_jobs(water3r, case, steps, warm, graph, gie_steps=2,
                                    labels=("gie_config3R", "gie_rmsnorm_config3R", "rmsnorm_config3R"))
            add("gie_config3R", "gie_zonal_scatter_fwd", jobs["gie"], water3r.n_edges, share=True)
            add("rmsnorm_config3R", "rmsnorm_fwd", jobs["rms"], jobs["rms"]["rows"], unit="rows/s", share=True)
            fused = add("gie_rmsnorm_config3R", "gie_zonal_scatter_rmsnorm_fwd", jobs["fused"], water3r.n_edges,
                        share=True)
            fused["unfused_ms_per_step"] = round(jobs["gie"]["ms_per_step"] + jobs["rms"]["ms_per_step"], 5)
            del jobs
            if backward:
                job = gie_backward_job(water3r, case, steps, warm, graph, gie_steps=2, label="gie_bwd_config3R")
                add("gie_bwd_config3R", "gie_zonal_scatter_bwd", job, job["edges"], share=True)
            del case
            torch.cuda.empty_cache()
            case = workloads.gie_config(water3r, seed=0, device="cuda", primary=False)
            jobs = gie_forward_jobs(water3r, case, steps, warm, graph, labels=("gie_config3R_secondary", None, None))
            add("gie_config3R_secondary", "gie_zonal_scatter_fwd", jobs["gie"], water3r.n_edges, share=True)
            if backward:
                job = gie_backward_job(water3r, case, steps, warm, graph, label="gie_bwd_config3R_secondary")
                add("gie_bwd_config3R_secondary", "gie_zonal_scatter_bwd", job, job["edges"], share=True)
                jobs = rmsnorm_jobs(114688, steps, warm, graph, labels=(None, "rmsnorm_bwd_config3R"))
                add("rmsnorm_bwd_config3R", "rmsnorm_bwd", jobs["bwd"], 114688, unit="rows/s", share=True)
            edges_3r = water3r.n_edges
            del case, water3r
            torch.cuda.empty_cache()
            progress("config 3R (primary, secondary) done")
            # ---- fused edge-stream chain over [E, 10, 64] at config 3R's edge count
            job = edge_stream_job(edges_3r, steps, warm, graph, label="edge_stream_combine_config3R")
            entry = add("edge_stream_combine_config3R", "edge_stream_combine", job, job["edges"], share=True)
            entry["torch_chain_ms_per_step"] = round(job["torch_chain_ms"], 5)
            del job
            torch.cuda.empty_cache()
            progress("edge stream chain done")
            jobs = rmsnorm_jobs(1048576, steps, warm, graph,
                                labels=("rmsnorm_rows1M", "rmsnorm_bwd_rows1M" if backward else None))
            add("rmsnorm_rows1M", "rmsnorm_fwd", jobs["fwd"], 1048576, unit="rows/s", share=True)
            if backward:
                add("rmsnorm_bwd_rows1M", "rmsnorm_bwd", jobs["bwd"], 1048576, unit="rows/s", share=True)
            del jobs
            torch.cuda.empty_cache()
            progress("rmsnorm 1M rows done")
        for key, op in ops.items():
            op["roofline"]["traffic"] = measured_traffic(key, op["roofline"]["algorithmic_bytes"])
        line["ops"] = ops
        if MARKS is None:
            line["reference_shapes"] = reference_shapes(steps)
            progress("reference latency shapes done")

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
    if MARKS is not None:
        line["traffic_marks"] = MARKS.labels

    if not args.no_cpu_baseline:
        progress("cpu baseline")
        headline_cpu, extras = cpu_baselines(head["base"], args.cpu_seconds, extra_cpu)
        line["cpu_baseline"] = headline_cpu
        for name, result in extras.items():
            if name in ops:
                ops[name]["cpu_baseline"] = result
    # the full line first, then the compact one the driver keeps (it stores the last ~8.5 KB of output)
    print(json.dumps({"detail": True, **line}), flush=True)
    print(json.dumps(compact_line(line)), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
