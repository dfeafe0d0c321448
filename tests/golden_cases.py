"""Loader of tests/golden/known_answers.json (the reference's known-answer cases).

Each case comes back with its lists turned into torch tensors of the right
dtype: lists of JSON integers as int64 (indices), ``*_f64`` expectations as
float64, other float lists as float32 (the dtype of the reference tests'
inputs; the generator writes every float with a decimal point).
"""
from __future__ import annotations

import json
from pathlib import Path

import torch

GOLDEN = Path(__file__).resolve().parent / "golden" / "known_answers.json"


def _leaves(value):
    if isinstance(value, list):
        for item in value:
            yield from _leaves(item)
    else:
        yield value


def _tensor(key: str, value):
    if value is None or not isinstance(value, list):
        return value
    if all(isinstance(leaf, int) for leaf in _leaves(value)):
        return torch.tensor(value, dtype=torch.int64)
    if key.endswith("_f64"):
        return torch.tensor(value, dtype=torch.float64)
    return torch.tensor(value, dtype=torch.float32)


def load_cases(op: str | None = None) -> list[dict]:
    cases = json.loads(GOLDEN.read_text())["cases"]
    out = []
    for case in cases:
        if op is not None and case["op"] != op:
            continue
        out.append({key: _tensor(key, value) for key, value in case.items()})
    return out


def case(name: str) -> dict:
    for item in load_cases():
        if item["name"] == name:
            return item
    raise KeyError(name)
