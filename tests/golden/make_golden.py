"""Writes tests/golden/known_answers.json -- the reference's known-answer cases.

Each case restates the inputs of a known-answer test of the reference
(lipengfei1409/bysj) and stores the expected outputs computed from the
mathematics, not from the oracle under test:

* exact-sum float64 loops (``oracle.loops``: ``math.fsum`` per element),
* a float32 edge-ordered loop in numpy for the sequential ``index_add_``
  arithmetic (bit-exact expectations),
* closed forms where the reference test states one (stable grouping,
  normalise-after-sum).

Inputs drawn from a torch generator in the reference tests are drawn here the
same way (``torch.Generator().manual_seed(s)``, ``torch.randn``), so the
fixture holds the same numbers; they are stored explicitly so that no
consumer depends on torch's RNG.  Float values are stored as JSON numbers
(float32 values are exactly representable as float64; ``repr`` round-trips).

Run from the repository root: ``python tests/golden/make_golden.py``.
"""
from __future__ import annotations

import json
import math
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import loops  # noqa: E402  (checker-side brute force, independent of oracle.segment)

OUT = Path(__file__).resolve().parent / "known_answers.json"


def _graph(sizes):
    """Destination-grouped edge list with the given per-node counts
    (tests/python/test_segment_ops_reference.py:21-27)."""
    dst = np.repeat(np.arange(len(sizes), dtype=np.int64), sizes)
    offsets = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    return dst, offsets


def _f32(values) -> list:
    return np.asarray(values, dtype=np.float32).astype(np.float64).tolist()


def _f64(values) -> list:
    return np.asarray(values, dtype=np.float64).tolist()


def _i64(values) -> list:
    return np.asarray(values, dtype=np.int64).tolist()


def csr_cases() -> list[dict]:
    """test_segment_ops_reference.py:31-45."""
    dst, offsets = _graph([2, 0, 3])
    src = np.array([2, 0, 2, 1, 0], dtype=np.int64)
    return [
        {"name": "offsets_2_0_3", "op": "segment_offsets", "dst": _i64(dst), "n_nodes": 3,
         "offsets": _i64(loops.offsets_loop(dst, 3)), "closed_form": [0, 2, 2, 5]},
        {"name": "group_by_source_stable", "op": "group_by_source", "src": _i64(src), "n_nodes": 3,
         "order": _i64(loops.stable_order_loop(src)), "offsets": _i64(loops.offsets_loop(src, 3)),
         "closed_form_order": [1, 4, 3, 0, 2], "closed_form_offsets": [0, 2, 3, 5]},
    ]


def segment_sum_cases() -> list[dict]:
    """test_segment_ops_reference.py:48-103."""
    cases = []
    dst, offsets = _graph([2, 1, 3])
    for label, src in (("arange", np.arange(12, dtype=np.float32).reshape(6, 2)),
                       ("arange_div7", (np.arange(12, dtype=np.float32) / np.float32(7)).reshape(6, 2))):
        edge_scale = torch.linspace(0.5, 1.5, 6).numpy()
        node_scale = np.array([1.0, 2.0, 3.0], dtype=np.float32)
        cases.append({
            "name": f"segment_sum_{label}", "op": "segment_sum", "dst": _i64(dst), "offsets": _i64(offsets),
            "src": _f32(src), "edge_scale": _f32(edge_scale), "node_scale": _f32(node_scale),
            "out_f64": _f64(loops.segment_sum_loop(src, dst, 3, edge_scale, node_scale)),
            "out_f32_sequential": _f32(loops.segment_sum_sequential_f32(src, dst, 3, edge_scale, node_scale)),
        })
    dst0, offsets0 = _graph([0, 2, 0])
    ones = np.ones((2, 3), dtype=np.float32)
    cases.append({
        "name": "segment_sum_empty_groups", "op": "segment_sum", "dst": _i64(dst0), "offsets": _i64(offsets0),
        "src": _f32(ones), "edge_scale": None, "node_scale": None,
        "out_f64": _f64(loops.segment_sum_loop(ones, dst0, 3)),
        "out_f32_sequential": _f32(loops.segment_sum_sequential_f32(ones, dst0, 3)),
        "closed_form": [[0, 0, 0], [2, 2, 2], [0, 0, 0]],
    })
    # Closed-form backward of test_segment_ops_reference.py:76-103, evaluated
    # element by element in float64 with exact sums.
    src = (np.arange(12, dtype=np.float32) / np.float32(7)).reshape(6, 2)
    edge_scale = torch.linspace(0.5, 1.5, 6).numpy()
    node_scale = np.array([1.0, 2.0, 3.0], dtype=np.float32)
    upstream = torch.randn(3, 2, generator=torch.Generator().manual_seed(11)).numpy()
    s64, w64, n64, g64 = (a.astype(np.float64) for a in (src, edge_scale, node_scale, upstream))
    grad_src = np.array([[g64[dst[e], c] * n64[dst[e]] * w64[e] for c in range(2)] for e in range(6)])
    grad_edge = np.array([math.fsum(g64[dst[e], c] * n64[dst[e]] * s64[e, c] for c in range(2)) for e in range(6)])
    prefix = loops.segment_sum_loop(src, dst, 3, edge_scale)
    grad_node = np.array([math.fsum(g64[n, c] * prefix[n, c] for c in range(2)) for n in range(3)])
    cases.append({
        "name": "segment_sum_backward_closed_form", "op": "segment_sum_backward", "dst": _i64(dst),
        "offsets": _i64(offsets), "src": _f32(src), "edge_scale": _f32(edge_scale), "node_scale": _f32(node_scale),
        "grad_out": _f32(upstream), "grad_src_f64": _f64(grad_src), "grad_edge_scale_f64": _f64(grad_edge),
        "grad_node_scale_f64": _f64(grad_node),
    })
    return cases


def segment_softmax_cases() -> list[dict]:
    """test_segment_ops_reference.py:106-185."""
    cases = []
    dst, offsets = _graph([2, 1, 3])
    env = np.array([0.9, -0.2, 0.7, 0.0, 1.1, 0.3], dtype=np.float32)
    for seed, null in ((0, True), (0, False)):
        generator = torch.Generator().manual_seed(seed)
        logit = torch.randn(6, 3, generator=generator).numpy()
        null_logit = torch.randn(3, 3, generator=generator).numpy() if null else None
        alpha, null_alpha = loops.segment_softmax_loop(logit, env, dst, 3, null_logit)
        cases.append({
            "name": f"segment_softmax_seed{seed}_{'null' if null else 'nonull'}", "op": "segment_softmax",
            "dst": _i64(dst), "offsets": _i64(offsets), "logit": _f32(logit), "env": _f32(env),
            "null_logit": None if null_logit is None else _f32(null_logit),
            "alpha_f64": _f64(alpha), "null_alpha_f64": None if null_alpha is None else _f64(null_alpha),
        })
    # Closed-form backward (test_segment_ops_reference.py:160-185): env made
    # positive as in the reference test, cotangents seeded.
    generator = torch.Generator().manual_seed(3)
    logit = torch.randn(6, 3, generator=generator).numpy()
    null_logit = torch.randn(3, 3, generator=generator).numpy()
    env_pos = np.abs(env)
    cot = torch.Generator().manual_seed(13)
    grad_alpha = torch.randn(6, 3, generator=cot).numpy()
    grad_null = torch.randn(3, 3, generator=cot).numpy()
    alpha, null_alpha = loops.segment_softmax_loop(logit, env_pos, dst, 3, null_logit)
    ga, gn = grad_alpha.astype(np.float64), grad_null.astype(np.float64)
    expectation = np.zeros((3, 3))
    for n in range(3):
        for c in range(3):
            terms = [alpha[e, c] * ga[e, c] for e in range(6) if dst[e] == n] + [null_alpha[n, c] * gn[n, c]]
            expectation[n, c] = math.fsum(terms)
    grad_logit = alpha * (ga - expectation[dst])
    grad_null_logit = null_alpha * (gn - expectation)
    env64 = env_pos.astype(np.float64)
    grad_env = np.array([math.fsum(grad_logit[e]) * (2.0 / env64[e] if env64[e] > 0 else 0.0) for e in range(6)])
    cases.append({
        "name": "segment_softmax_backward_closed_form", "op": "segment_softmax_backward", "dst": _i64(dst),
        "offsets": _i64(offsets), "logit": _f32(logit), "env": _f32(env_pos), "null_logit": _f32(null_logit),
        "grad_alpha": _f32(grad_alpha), "grad_null_alpha": _f32(grad_null),
        "grad_logit_f64": _f64(grad_logit), "grad_null_logit_f64": _f64(grad_null_logit),
        "grad_env_f64": _f64(grad_env),
    })
    return cases


def force_cases() -> list[dict]:
    """test_segment_ops_reference.py:188-225."""
    cases = []
    dst, dst_offsets = _graph([2, 1, 3])
    src = np.array([2, 0, 2, 1, 0, 2], dtype=np.int64)
    for seed in (0, 1):
        generator = torch.Generator().manual_seed(seed)
        grad_edge = torch.randn(6, 3, generator=generator).numpy()
        edge_vec = torch.randn(6, 3, generator=generator).numpy()
        force, virial = loops.force_assembly_loop(grad_edge, edge_vec, src, dst, 3)
        cases.append({
            "name": f"force_assembly_seed{seed}", "op": "force_assembly", "dst": _i64(dst),
            "dst_offsets": _i64(dst_offsets), "src": _i64(src),
            "src_order": _i64(loops.stable_order_loop(src)), "src_offsets": _i64(loops.offsets_loop(src, 3)),
            "grad_edge": _f32(grad_edge), "edge_vec": _f32(edge_vec),
            "force_f64": _f64(force), "virial_f64": _f64(virial),
        })
    return cases


def gie_cases() -> list[dict]:
    """tests/python/test_gie.py:19-30, 69-103 and 180-189."""
    zonal = np.array([[0.2, -0.1, 0.3], [0.4, 0.5, -0.2], [-0.3, 0.6, 0.1], [0.7, -0.2, 0.4]], dtype=np.float32)
    radial = (np.arange(24, dtype=np.float32) / np.float32(10)).reshape(4, 2, 3)
    dst = np.array([1, 0, 1, 1], dtype=np.int64)
    slots = np.array([0, 0, 1], dtype=np.int64)
    inverse = np.array([0.7, 0.5], dtype=np.float32)
    cases = [{
        "name": "gie_fixture", "op": "zonal_scatter", "zonal": _f32(zonal), "radial": _f32(radial),
        "dst": _i64(dst), "radial_slot": _i64(slots), "inv_sqrt_deg": _f32(inverse),
        "out_f64": _f64(loops.zonal_scatter_loop(zonal, radial, dst, slots, inverse)),
    }]
    # Normalise after the destination sum: the float32 sum in edge order is
    # (1e8 + (-1e8 + 8)) + 1 = 9 exactly, then one rounding of 9 * 0.3.
    big = np.array([[1e8], [-1e8 + 8], [1.0]], dtype=np.float32)
    exact = np.float32(np.float32(np.float32(big[0, 0] + big[1, 0]) + big[2, 0]) * np.float32(0.3))
    cases.append({
        "name": "gie_normalise_after_sum", "op": "zonal_scatter", "zonal": _f32(big),
        "radial": _f32(np.ones((3, 1, 1), dtype=np.float32)), "dst": [0, 0, 0], "radial_slot": [0],
        "inv_sqrt_deg": _f32([0.3]), "exact_f32_row1": _f32([exact]),
        "out_f64": _f64(loops.zonal_scatter_loop(big, np.ones((3, 1, 1), np.float32), [0, 0, 0], [0], [0.3])),
    })
    return cases


def gie_backward_cases() -> list[dict]:
    """Gradients of the test_gie.py fixture (tests/python/test_gie.py:19-30, 135-166).

    The reference checks its backward against autograd of the forward chain
    with an unseeded upstream of shape [2, 4, 3]; here the upstream is seeded
    and the expectation is the closed form (``loops.zonal_scatter_backward_loop``),
    with radial_slot = [0, 0, 1] so slot 0 is shared by rows 0 and 1 and its
    gradient is a sum over both.  A second case takes the inverse degree as
    [N, 1, 1] and a wider, irregular graph with an empty node and an
    unreferenced radial slot (its gradient must be zero).
    """
    zonal = np.array([[0.2, -0.1, 0.3], [0.4, 0.5, -0.2], [-0.3, 0.6, 0.1], [0.7, -0.2, 0.4]], dtype=np.float32)
    radial = (np.arange(24, dtype=np.float32) / np.float32(10)).reshape(4, 2, 3)
    dst = np.array([1, 0, 1, 1], dtype=np.int64)
    slots = np.array([0, 0, 1], dtype=np.int64)
    inverse = np.array([0.7, 0.5], dtype=np.float32)
    upstream = torch.randn(2, 4, 3, generator=torch.Generator().manual_seed(17)).numpy()
    gz, gr, gi = loops.zonal_scatter_backward_loop(upstream, zonal, radial, dst, slots, inverse)
    cases = [{
        "name": "gie_backward_fixture", "op": "zonal_scatter_backward", "grad_output": _f32(upstream),
        "zonal": _f32(zonal), "radial": _f32(radial), "dst": _i64(dst), "radial_slot": _i64(slots),
        "inv_sqrt_deg": _f32(inverse), "grad_zonal_f64": _f64(gz), "grad_radial_f64": _f64(gr),
        "grad_inv_sqrt_deg_f64": _f64(gi),
    }]
    generator = torch.Generator().manual_seed(23)
    n_nodes, n_edges, n_rows, n_radial, channels = 5, 11, 4, 4, 2
    dst = torch.randint(0, n_nodes - 1, (n_edges,), generator=generator).numpy()  # node 4 has no edge
    zonal = torch.randn(n_edges, n_rows, generator=generator).numpy()
    radial = torch.randn(n_edges, n_radial, channels, generator=generator).numpy()
    slots = np.array([2, 0, 2, 1], dtype=np.int64)  # slot 2 shared, slot 3 unreferenced
    inverse = (torch.rand(n_nodes, generator=generator) + 0.25).numpy().reshape(n_nodes, 1, 1)
    upstream = torch.randn(n_nodes, n_rows + 1, channels, generator=generator).numpy()
    gz, gr, gi = loops.zonal_scatter_backward_loop(upstream, zonal, radial, dst, slots, inverse)
    cases.append({
        "name": "gie_backward_shared_and_unreferenced_slots", "op": "zonal_scatter_backward",
        "grad_output": _f32(upstream), "zonal": _f32(zonal), "radial": _f32(radial), "dst": _i64(dst),
        "radial_slot": _i64(slots), "inv_sqrt_deg": _f32(inverse), "grad_zonal_f64": _f64(gz),
        "grad_radial_f64": _f64(gr), "grad_inv_sqrt_deg_f64": _f64(gi),
    })
    return cases


def rmsnorm_cases() -> list[dict]:
    """tests/python/test_rmsnorm.py:61-80."""
    generator = torch.Generator().manual_seed(5)
    x = torch.randn(3, 2, 17, generator=generator).numpy()
    scale = torch.randn(17, generator=generator).numpy()
    return [
        {"name": "rmsnorm_random", "op": "rmsnorm", "x": _f32(x), "scale": _f32(scale), "eps": 1e-5,
         "out_f64": _f64(loops.rmsnorm_loop(x, scale, 1e-5))},
        {"name": "rmsnorm_zeros", "op": "rmsnorm", "x": _f32(np.zeros((2, 7), np.float32)), "scale": None,
         "eps": 1e-6, "out_f64": _f64(np.zeros((2, 7)))},
    ]


def main() -> None:
    cases = csr_cases() + segment_sum_cases() + segment_softmax_cases() + force_cases() + gie_cases() \
        + gie_backward_cases() + rmsnorm_cases()
    payload = {"source": "lipengfei1409/bysj tests/python known-answer cases; expectations from exact-sum loops",
               "cases": cases}
    lines = ",\n".join(json.dumps(case, separators=(",", ":")) for case in cases)
    OUT.write_text('{"source":' + json.dumps(payload["source"]) + ',\n"cases":[\n' + lines + "\n]}\n")
    print(f"wrote {len(cases)} cases to {OUT.relative_to(ROOT)}")


if __name__ == "__main__":
    main()
