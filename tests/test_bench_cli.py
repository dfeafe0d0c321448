"""bench.py's command-line contract on the CPU: one GPU only, and a loud failure without one."""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]


def _bench(*args: str) -> subprocess.CompletedProcess:
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True, text=True,
                          timeout=300, cwd=ROOT)


def test_more_than_one_gpu_is_refused_with_a_message():
    result = _bench("--gpus", "2", "--steps", "1", "--warmup", "0")
    assert result.returncode == 2
    assert "one GPU" in result.stderr
    assert result.stdout == ""


@pytest.mark.skipif(torch.cuda.is_available(), reason="a GPU is visible")
def test_without_a_gpu_the_bench_fails_instead_of_measuring_the_cpu():
    result = _bench("--steps", "1", "--warmup", "0")
    assert result.returncode == 1
    assert "gfx950" in result.stderr
    assert result.stdout == ""


# ---------------------------------------------------------------------------
# --traffic-summary: the counter CSVs of two rocprofv3 --pmc passes -> traffic per bench line
# ---------------------------------------------------------------------------

_HEADER = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id", "Thread_Id", "Grid_Size",
           "Kernel_Id", "Kernel_Name", "Workgroup_Size", "LDS_Block_Size", "Scratch_Size", "VGPR_Count",
           "Accum_VGPR_Count", "SGPR_Count", "Counter_Name", "Counter_Value", "Start_Timestamp", "End_Timestamp"]
_MARKER = "void dpa4k::(anonymous namespace)::stream_read_kernel(float const*, long, float*)"
_COPY = "void dpa4k::(anonymous namespace)::stream_copy_kernel(float const*, long, float*, long)"
_SOFTMAX = "void dpa4k::softmax_forward_kernel<4, 1, true, false, true>(float const*, float const*)"
_FILL = "void at::native::vectorized_elementwise_kernel<4, at::native::FillFunctor<float>>(int, float*)"


def _write_counters(path, counter, dispatches):
    """dispatches: (kernel name, workgroups, counter value in KiB), in launch order."""
    import csv

    with open(path, "w", newline="") as handle:
        writer = csv.writer(handle)
        writer.writerow(_HEADER)
        for i, (name, blocks, value) in enumerate(dispatches, start=1):
            writer.writerow([i, i, "Agent 1", 1, 1, 1, blocks * 256, 7, name, 256, 0, 0, 32, 0, 16, counter,
                             value, 0, 1])


def _dispatch_list(step_values, calibration_kib, setup_kib):
    """A marked dispatch list: the calibration line (label 0), then one line (label 1) of three steps."""
    out = [(_SOFTMAX, 100, 999.0),  # before any line: ignored
           (_MARKER, 3, 0.0), (_MARKER, 1, 0.0), (_COPY, 8192, calibration_kib), (_MARKER, 2, 0.0),
           (_MARKER, 4, 0.0), (_FILL, 10, setup_kib)]  # set-up launch before the first step: ignored
    for kernel_kib, fill_kib in step_values:
        out += [(_MARKER, 1, 0.0), (_SOFTMAX, 64, kernel_kib), (_FILL, 10, fill_kib)]
    out += [(_MARKER, 2, 0.0), (_SOFTMAX, 100, 555.0)]  # after the line closes: ignored
    return out


def _traffic_case(tmp_path, write_steps=None):
    import json

    fetch = tmp_path / "fetch.csv"
    write = tmp_path / "write.csv"
    # FETCH counts a 256 MiB copy as 128 MiB (scale 2), WRITE counts it in full (scale 1)
    _write_counters(fetch, "FETCH_SIZE", _dispatch_list([(5000.0, 1.0), (1000.0, 3.0), (1200.0, 1.0)],
                                                        131072.0, 7.0))
    _write_counters(write, "WRITE_SIZE", write_steps or _dispatch_list([(9.0, 1.0), (700.0, 4.0), (500.0, 2.0)],
                                                                       262144.0, 7.0))
    log = tmp_path / "fetch.log"
    line = {"config": {"workload": "segment_softmax_fwd_config2"},
            "roofline": {"algorithmic_bytes": 4_000_000}, "ops": {},
            "traffic_marks": ["calibration_copy", "segment_softmax_fwd_config2"]}
    log.write_text("[bench] progress on stderr\n" + json.dumps(line) + "\n")
    return fetch, write, log


def test_traffic_summary_prices_each_marked_step(tmp_path):
    import json

    import bench

    fetch, write, log = _traffic_case(tmp_path)
    assert bench.traffic_summary(str(fetch), str(write), str(log), out_dir=tmp_path) == 0
    entry = json.loads((tmp_path / "traffic.json").read_text())["segment_softmax_fwd_config2"]
    assert entry["fetch_scale"] == 2.0 and entry["write_scale"] == 1.0
    # steps after the first: fetch (1000 + 3) and (1200 + 1) KiB -> median 1102 KiB, x2 scale
    assert entry["fetch_bytes"] == int(1102.0 * 1024 * 2)
    # write (700 + 4) and (500 + 2) KiB -> median 603 KiB
    assert entry["write_bytes"] == int(603.0 * 1024)
    assert entry["bytes_per_launch"] == int(1102.0 * 1024 * 2 + 603.0 * 1024)
    assert entry["algorithmic_bytes"] == 4_000_000 and entry["steps"] == 2
    assert entry["kernels"] == ["dpa4k::softmax_forward_kernel<4, 1, true, false, true>",
                                "at::native::vectorized_elementwise_kernel<4, at::native::FillFunctor<float>>"]
    assert "calibration_copy" not in json.loads((tmp_path / "traffic.json").read_text())
    table = (tmp_path / "traffic.md").read_text()
    assert "rocprofv3 --pmc FETCH_SIZE" in table and "| segment_softmax_fwd_config2 |" in table


def test_traffic_summary_refuses_passes_that_launched_different_kernels(tmp_path):
    import bench

    other = _dispatch_list([(9.0, 1.0), (700.0, 4.0), (500.0, 2.0)], 262144.0, 7.0)
    other[-3] = (_SOFTMAX, 65, 500.0)  # the last step of the line launches another kernel
    fetch, write, log = _traffic_case(tmp_path, write_steps=other)
    with pytest.raises(SystemExit, match="different kernels"):
        bench.traffic_summary(str(fetch), str(write), str(log), out_dir=tmp_path)


# ---------------------------------------------------------------------------
# the final line: every op row inside what the driver keeps
# ---------------------------------------------------------------------------

def _full_line(n_ops: int) -> dict:
    roof = {"bound": "hbm", "achieved": 5656.2, "peak": 8000.0, "unit": "GB/s", "frac": 0.707, "traffic": 5_600_000_000,
            "algorithmic_bytes": 5_503_000_000}
    op = {"op": "segment_sum_fwd", "value": 10771234567.8, "unit": "edges/s", "ms_per_step": 0.97308, "input_sets": 3,
          "roofline": roof, "edges": 10485760, "nodes": 262144, "channels": 128, "same_bytes_copy_us": 1041.9,
          "share_of_same_bytes_copy": 1.0707,
          "cpu_baseline": {"value": 2.7e7, "unit": "edges/s", "cores": 16, "sample": "x" * 120, "ms_per_call": 213.4}}
    shapes = {f"shape_{i}": {"eager_ms": 0.0235, "kernel_ms": 0.0232, "torch_gpu_ms": 0.4899, "dcu_ms": 0.49,
                             "dcu_torch_ms": 4.42, "source": "docs/task2-hip-fusion-plan.md:229"} for i in range(6)}
    shapes["rmsnorm_1x128"] = {"eager_median_us": 9.9, "eager_p95_us": 10.2, "kernel_us": 1.9, "dcu_ms": None,
                               "source": "tests/csrc/latency/test_rmsnorm_latency.py"}
    shapes["note"] = "same inputs every call" * 5
    return {"metric": "segment-op edges/s + % HBM roofline (segment_softmax forward, config 2)", "value": 5.7e10,
            "unit": "edges/s", "n_gpus": 1, "steps": 20, "warmup": 5, "ms_per_step": 0.01516,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
            "config": {"workload": "segment_softmax_fwd_config2"}, "roofline": dict(roof),
            "stream_ceilings": {"read_GBps": 6038.8, "note": "n" * 200},
            "ops": {f"op_with_a_long_name_{i:02d}": dict(op) for i in range(n_ops)}, "reference_shapes": shapes,
            "config5_dpa4_end_to_end": {"status": "unavailable", "unit": "atom-steps/s", "value": None,
                                        "reason": "r" * 200},
            "cpu_baseline": {"value": 6.4e7, "unit": "edges/s", "cores": 16, "kind": "port", "sample": "s" * 150}}


def test_final_line_keeps_every_op_within_the_drivers_tail():
    import json

    import bench

    line = _full_line(40)  # more ops than the default run prints (31)
    assert len(json.dumps(line)) > 2 * bench.FINAL_LINE_LIMIT
    final = bench.compact_line(line)
    text = json.dumps(final)
    assert len(text) < bench.FINAL_LINE_LIMIT
    assert set(final["ops"]) == set(line["ops"])
    row = dict(zip(final["ops_fields"], final["ops"]["op_with_a_long_name_07"]))
    assert row["frac"] == 0.707 and row["unit"] == "edges/s" and row["us_per_step"] == 973.08
    assert row["traffic_over_algorithmic"] == round(5_600_000_000 / 5_503_000_000, 3)
    assert row["share_of_same_bytes_copy"] == 1.0707 and row["achieved_GBps"] == 5656
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "roofline", "cpu_baseline"):
        assert final[key] == line[key]
    shapes = dict(zip(final["reference_shapes_fields"], final["reference_shapes"]["rmsnorm_1x128"]))
    assert shapes["eager_ms"] == 0.0099 and shapes["kernel_ms"] == 0.0019
    assert final["config5_dpa4_end_to_end"]["status"] == "unavailable"


def test_traffic_summary_reads_the_detail_line(tmp_path):
    import json

    import bench

    detail = {"detail": True, "config": {"workload": "w"}, "roofline": {"algorithmic_bytes": 7}, "ops": {}}
    log = tmp_path / "bench.log"
    log.write_text(json.dumps(detail) + "\n" + json.dumps({"ops": {"x": [1, 2]}}) + "\n")
    assert bench._bench_json(str(log)) == detail


def test_trace_summary_lists_library_kernels_and_the_bench_lines(tmp_path):
    import csv
    import json

    import bench

    stats, trace, log = tmp_path / "stats.csv", tmp_path / "trace.csv", tmp_path / "bench.log"
    with open(stats, "w", newline="") as handle:
        writer = csv.writer(handle)
        writer.writerow(["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs", "MaxNs", "StdDev"])
        writer.writerow([_SOFTMAX, 24, 340000, 14166.7, 50.0, 14000, 14500, 10])
        writer.writerow([_FILL, 3, 300, 100, 1.0, 90, 110, 1])
    with open(trace, "w", newline="") as handle:
        writer = csv.writer(handle)
        writer.writerow(["Kernel_Name", "Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z", "Start_Timestamp",
                         "End_Timestamp"])
        for i in range(24):
            writer.writerow([_SOFTMAX, 16384, 1, 1, 1000 * i, 1000 * i + 14000 + i])
    detail = {"detail": True, "config": {"workload": "segment_softmax_fwd_config2"}, "ms_per_step": 0.01514,
              "roofline": {"frac": 0.49}, "ops": {"segment_sum_config1": {"ms_per_step": 0.0111,
                                                                          "roofline": {"frac": 0.24}}}}
    log.write_text(json.dumps(detail) + "\n" + json.dumps({"ops": {}}) + "\n")
    assert bench.trace_summary(str(stats), str(trace), str(log), out_dir=tmp_path) == 0
    text = (tmp_path / "all_ops_kernel_stats.md").read_text()
    assert "| `dpa4k::softmax_forward_kernel<4, 1, true, false, true>` | 24 | 14167 |" in text
    assert "FillFunctor" not in text  # torch kernels are not listed
    assert "| `dpa4k::softmax_forward_kernel<4, 1, true, false, true>` | 16,384 | 24 | 14.0 |" in text
    assert "| segment_softmax_fwd_config2 (headline) | 15.14 | 0.49 |" in text
    assert "| segment_sum_config1 | 11.10 | 0.24 |" in text
    assert bench.TRACE_COMMAND in text


def test_counter_table_gives_each_kernels_median_per_counter(tmp_path):
    import bench

    first, second = tmp_path / "a.csv", tmp_path / "b.csv"
    _write_counters(first, "SQ_WAVES", [(_SOFTMAX, 64, 10.0), (_SOFTMAX, 64, 30.0), (_SOFTMAX, 64, 20.0),
                                        (_FILL, 10, 5.0)])
    _write_counters(second, "GRBM_GUI_ACTIVE", [(_SOFTMAX, 64, 1000.0), (_SOFTMAX, 64, 3000.0)])
    table = bench.counter_table([str(first), str(second)])
    lines = table.splitlines()
    assert lines[0] == "| Kernel | Dispatches | GRBM_GUI_ACTIVE | SQ_WAVES |"
    assert "| `dpa4k::softmax_forward_kernel<4, 1, true, false, true>` | 3 | 2,000 | 20 |" in lines
    assert any(line.startswith("| `at::native::vectorized_elementwise_kernel") and line.endswith("|  | 5 |")
               for line in lines)
