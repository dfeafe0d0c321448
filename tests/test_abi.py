"""The C ABI of libdpa4k.so on the CPU: it loads, and it exports what include/dpa4k.h declares.

No compute call is made (there is no GPU here).  Only entry points whose
argument checks return before any HIP call are exercised: the version and
error queries, the workspace-size queries, and the EINVAL paths for sizes a
caller must never pass.
"""
from __future__ import annotations

import ctypes
import re
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "dpa4k.h"
LIBRARY = ROOT / "bysj_amd" / "libdpa4k.so"

pytestmark = pytest.mark.skipif(not LIBRARY.exists(), reason="libdpa4k.so is not built (run __graft_entry__.build())")


def _declarations() -> dict[str, int]:
    """name -> parameter count of every function declared in the header."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    found = {}
    for match in re.finditer(r"\b(dpa4k_\w+)\s*\(([^)]*)\)\s*;", text):
        params = match.group(2).strip()
        found[match.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return found


def _lib():
    from bysj_amd.kernels import _lib

    return _lib


def test_header_and_binding_declare_the_same_entry_points():
    declared = _declarations()
    prototypes = _lib().PROTOTYPES
    assert set(declared) == set(prototypes), set(declared) ^ set(prototypes)
    for name, count in declared.items():
        assert len(prototypes[name][1]) == count, f"{name}: header has {count} parameters"


def test_library_exports_every_declared_symbol():
    exported = subprocess.run(["nm", "-D", "--defined-only", str(LIBRARY)], capture_output=True, text=True,
                              check=True).stdout
    names = {line.split()[-1] for line in exported.splitlines() if line.strip()}
    missing = sorted(set(_declarations()) - names)
    assert not missing, f"not exported: {missing}"
    dpa4k_exports = sorted(n for n in names if n.startswith("dpa4k_"))
    assert set(dpa4k_exports) == set(_declarations()), "exports beyond the header"


def test_library_loads_and_reports_its_abi_version():
    lib = _lib().load()
    version = int(re.search(r"#define DPA4K_ABI_VERSION (\d+)", HEADER.read_text()).group(1))
    assert lib.dpa4k_abi_version() == version == _lib().ABI_VERSION
    assert lib.dpa4k_last_error() == b""


def test_workspace_queries_are_host_only_and_grow_with_the_input():
    lib = _lib().load()
    for query in ("dpa4k_segment_offsets_workspace_size", "dpa4k_group_by_key_workspace_size",
                  "dpa4k_gie_group_workspace_size", "dpa4k_gie_workspace_size",
                  "dpa4k_rmsnorm_backward_workspace_size"):
        function = getattr(lib, query)
        small, large = function(1000, 100), function(10_000_000, 100_000)
        assert large >= small, query
        assert large % 256 == 0 or large == 0, f"{query}: carve granularity"


def test_invalid_sizes_fail_before_any_device_call():
    binding = _lib()
    lib = binding.load()
    null = None
    cases = [
        (lib.dpa4k_segment_sum_forward, (null,) * 6 + (-1, 1, 1, null), "negative sizes"),
        (lib.dpa4k_segment_sum_forward, (null,) * 6 + (1, 1, 0, null), "at least one channel"),
        (lib.dpa4k_segment_softmax_forward, (null,) * 7 + (-1, 1, 1, null), ""),
        (lib.dpa4k_rmsnorm_forward, (null,) * 4 + (1, 0, ctypes.c_float(1e-6), null), "feature dimension"),
        (lib.dpa4k_rmsnorm_forward, (null,) * 4 + (1, 4, ctypes.c_float(0.0), null), "eps"),
        (lib.dpa4k_force_assembly_f32, (null,) * 7 + (0, 0, null), ""),
        (lib.dpa4k_force_assembly_f64, (null,) * 7 + (-1, 1, null), ""),
        # a scale gradient needs a scale (csrc/rmsnorm.cpp:138-139 of the reference); the output
        # pointer is never dereferenced
        (lib.dpa4k_rmsnorm_backward, (null,) * 5 + (ctypes.c_void_p(256), 1, 4, null, 0, null),
         "scale is omitted"),
        # beyond what rows of blocks along y can hold
        (lib.dpa4k_segment_sum_forward, (null,) * 6 + (1, 2**62, 1, null), "segment count too large"),
        (lib.dpa4k_segment_softmax_forward, (null,) * 7 + (1, 2**62, 8, null), "segment count too large"),
        (lib.dpa4k_rmsnorm_forward, (null,) * 4 + (2**62, 4, ctypes.c_float(1e-6), null), "launch limit"),
        (lib.dpa4k_gie_zonal_scatter_forward_csr, (null,) * 7 + (0, 2**62, 0, 0, 4, 0, null), "launch limit"),
        (lib.dpa4k_force_assembly_f32, (null,) * 7 + (0, 2**62, null), "launch limit"),
        (lib.dpa4k_edge_stream_combine, (null,) * 3 + (0, 0) + (null,) * 3 + (1, 1, 1, null), "1 to 4 terms"),
        (lib.dpa4k_edge_stream_combine, (null,) * 3 + (1, 7) + (null,) * 3 + (1, 1, 1, null), "unknown activation"),
        (lib.dpa4k_edge_stream_combine, (null,) * 3 + (1, 0) + (null,) * 3 + (2**40, 2**20, 2**10, null),
         "overflows 64 bits"),
    ]
    for function, args, fragment in cases:
        status = function(*args)
        assert status == binding.EINVAL, (function.__name__, status)
        message = lib.dpa4k_last_error().decode()
        assert message and fragment in message, (function.__name__, message)


def test_package_imports_under_the_reference_names():
    """With bysj_amd/ on sys.path the operators import as the reference's `kernels` package."""
    code = (
        "import sys; sys.path.insert(0, %r)\n"
        "import kernels, kernels._C as native\n"
        "print(','.join(kernels.__all__)); print(native.segment_sum_forward.__module__)\n"
    ) % str(ROOT / "bysj_amd")
    result = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert result.returncode == 0, result.stderr
    names, module = result.stdout.strip().splitlines()
    assert names.split(",") == [
        "force_assembly", "gie_available", "gie_zonal_scatter", "group_by_source", "rmsnorm",
        "rmsnorm_available", "segment_available", "segment_offsets", "segment_softmax", "segment_sum",
        "zonal_scatter",
    ]
    assert module == "kernels._C"


def test_launch_row_limit_hook():
    binding = _lib()
    lib = binding.load()
    assert lib.dpa4k_set_launch_row_limit(-1) == binding.EINVAL
    assert "non-negative" in lib.dpa4k_last_error().decode()
    args = (None,) * 6 + (1, 2**40, 1, None)
    # 2^40 segments fit in 65,536 rows of the hardware limit (the call then stops at its null pointers) ...
    assert lib.dpa4k_segment_sum_forward(*args) == binding.EINVAL
    assert "null pointer" in lib.dpa4k_last_error().decode()
    # ... but not in rows of 3 blocks
    assert lib.dpa4k_set_launch_row_limit(3) == binding.OK
    try:
        assert lib.dpa4k_segment_sum_forward(*args) == binding.EINVAL
        assert "segment count too large" in lib.dpa4k_last_error().decode()
    finally:
        assert lib.dpa4k_set_launch_row_limit(0) == binding.OK


def test_softmax_plan_is_refused_for_other_offsets():
    """A plan lists the long segments of the offsets it was built from; other offsets of the same size are refused."""
    import torch

    from bysj_amd.kernels import _C

    offsets = torch.tensor([0, 3, 9, 10], dtype=torch.int64)
    plan = _C.SoftmaxPlan(torch.zeros(4, dtype=torch.int32), 0, 96, 10, 8, _C._offsets_fingerprint(offsets))
    assert _C._plan_args(plan, offsets, 10, 8) is plan
    assert _C._plan_args(None, offsets, 10, 8) is None
    same_values = offsets.clone()  # equal values, other storage
    with pytest.raises(RuntimeError, match="another graph"):
        _C._plan_args(plan, same_values, 10, 8)
    with pytest.raises(RuntimeError, match="another graph"):
        _C._plan_args(plan, offsets, 10, 4)  # another channel count
    offsets[1] = 5  # an in-place write bumps the version counter
    with pytest.raises(RuntimeError, match="another graph"):
        _C._plan_args(plan, offsets, 10, 8)
    with torch.inference_mode():
        frozen = torch.tensor([0, 3, 9, 10], dtype=torch.int64)
    frozen_plan = _C.SoftmaxPlan(plan.words, 0, 96, 10, 8, _C._offsets_fingerprint(frozen))
    assert _C._plan_args(frozen_plan, frozen, 10, 8) is frozen_plan


def test_plans_are_refused_for_a_new_tensor_at_a_freed_tensors_address():
    """A plan holds its graph tensors weakly: a same-size graph allocated where a freed one was is refused."""
    import gc

    import torch

    from bysj_amd.kernels import _C

    offsets = torch.tensor([0, 3, 9, 10], dtype=torch.int64)
    plan = _C.SoftmaxPlan(torch.zeros(4, dtype=torch.int32), 0, 96, 10, 8, _C._offsets_fingerprint(offsets))
    stamp = plan.fingerprint.stamp
    del offsets
    gc.collect()
    reused = torch.tensor([0, 1, 2, 10], dtype=torch.int64)
    # whether or not the allocator hands back the same address, a stamp of the same
    # address, size and version held by a dead reference must not match
    plan.fingerprint.stamp = _C._TensorStamp._stamp_of(reused)
    assert plan.fingerprint.ref() is None and stamp[1:] == plan.fingerprint.stamp[1:]
    with pytest.raises(RuntimeError, match="another graph"):
        _C._plan_args(plan, reused, 10, 8)
    graph = [torch.tensor([0, 2, 5], dtype=torch.int64), torch.tensor([0, 4, 5], dtype=torch.int64),
             torch.arange(5, dtype=torch.int64)]
    stamps = _C._force_fingerprint(*graph)
    holder = _C.ForcePlan(torch.zeros(1), torch.zeros(1), 5, 2, 4, 1, 1, stamps)
    assert _C._force_plan_matches(holder, *graph)
    assert not _C._force_plan_matches(holder, graph[0], graph[1], graph[2].clone())
