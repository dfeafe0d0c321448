"""Parity assertions shared by the test modules.

fp32 rule (the reference's, tests/csrc/accuracy/test_segment_ops_accuracy.py:140-144,
and BASELINE north_star): |actual - expected| <= 1e-5 * |expected| + 1e-5 * max|expected|,
checked against the fp32 oracle and against an fp64 ground truth.  fp64 rule:
the same with 1e-12.  Index results are compared bit for bit.
"""
from __future__ import annotations

import numpy as np
import torch

FP32_RTOL = 1e-5
FP32_SCALE = 1e-5
FP64_RTOL = 1e-12
FP64_SCALE = 1e-12


def _as64(value) -> np.ndarray:
    if isinstance(value, torch.Tensor):
        value = value.detach().cpu().double().numpy()
    return np.asarray(value, dtype=np.float64)


def assert_close_scaled(actual, expected, *, rtol=FP32_RTOL, scale=FP32_SCALE, what="") -> None:
    a, e = _as64(actual), _as64(expected)
    assert a.shape == e.shape, f"{what}: shape {a.shape} != {e.shape}"
    if e.size == 0:
        return
    both_nan = np.isnan(a) & np.isnan(e)
    budget = rtol * np.abs(e) + scale * np.nanmax(np.abs(e))
    error = np.abs(a - e)
    bad = ~(both_nan | (error <= budget))
    if bad.any():
        index = np.unravel_index(np.argmax(np.where(bad, error - budget, -np.inf)), a.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {a.size} elements outside |d| <= {rtol}|ref| + {scale} max|ref|; "
            f"worst at {index}: actual {a[index]!r} expected {e[index]!r}"
        )


def assert_gradient(actual, oracle, truth, what="") -> None:
    """A float32 gradient against the fp32 oracle and the fp64 closed form, each at the fp32 rule."""
    assert_close_scaled(actual, truth, what=f"{what} vs fp64 truth")
    assert_close_scaled(actual, oracle, what=f"{what} vs fp32 oracle")


def assert_fp64(actual, expected, what="") -> None:
    assert_close_scaled(actual, expected, rtol=FP64_RTOL, scale=FP64_SCALE, what=what)


def assert_bitwise(actual, expected, what="") -> None:
    a = actual.detach().cpu() if isinstance(actual, torch.Tensor) else torch.as_tensor(actual)
    e = expected.detach().cpu() if isinstance(expected, torch.Tensor) else torch.as_tensor(expected)
    assert a.shape == e.shape, f"{what}: shape {tuple(a.shape)} != {tuple(e.shape)}"
    if a.dtype.is_floating_point:
        same = (a == e) | (torch.isnan(a) & torch.isnan(e))
    else:
        same = a == e
    if not bool(same.all()):
        mismatch = int((~same).sum())
        raise AssertionError(f"{what}: {mismatch} of {a.numel()} elements differ bitwise")


def announce(*parts) -> None:
    """Name the case on stdout before a GPU step (so a lost box still names it)."""
    print("[case]", *parts, flush=True)
