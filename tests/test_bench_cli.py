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
