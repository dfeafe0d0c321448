"""The gfx950 path against the reference's known-answer cases (tests/golden/known_answers.json).

The same checks that pin the CPU oracle (test_oracle_pinning.py) run here on
the operators in kernels.* -> libdpa4k.so, with inputs copied to cuda:0 and
results copied back: bit-exact where the expectation is an integer or the
sequential float32 sum, the fp32 rule against the exact-sum expectations
otherwise.
"""
from __future__ import annotations

import pytest
import torch

from bysj_amd import kernels
from parity import announce
from test_oracle_pinning import (
    check_force,
    check_gie,
    check_offsets,
    check_rmsnorm,
    check_segment_softmax,
    check_segment_softmax_backward,
    check_segment_sum,
    check_segment_sum_backward,
)

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _dev(t):
    return None if t is None else t.to(DEV)


def _leaf(t):
    return None if t is None else t.to(DEV).requires_grad_(True)


def test_csr_helpers_golden():
    announce("golden csr")
    check_offsets(lambda d, n: kernels.segment_offsets(_dev(d), n).cpu(),
                  lambda s, n: tuple(t.cpu() for t in kernels.group_by_source(_dev(s), n)))


def test_segment_sum_golden():
    announce("golden segment_sum")

    def run(src, dst, offsets, w, s):
        return kernels.segment_sum(_dev(src), _dev(dst), _dev(offsets), _dev(w), _dev(s)).cpu()

    check_segment_sum(run)

    def backward(grad_out, src, dst, offsets, w, s):
        leaves = (_leaf(src), _leaf(w), _leaf(s))
        out = kernels.segment_sum(leaves[0], _dev(dst), _dev(offsets), leaves[1], leaves[2])
        return tuple(g.cpu() for g in torch.autograd.grad(out, leaves, _dev(grad_out)))

    check_segment_sum_backward(backward)


def test_segment_softmax_golden():
    announce("golden segment_softmax")

    def run(logit, env, dst, offsets, null):
        result = kernels.segment_softmax(_dev(logit), _dev(env), _dev(offsets), _dev(null))
        if null is None:
            return result.cpu(), None
        return result[0].cpu(), result[1].cpu()

    check_segment_softmax(run)

    def backward(grad_alpha, logit, env, dst, offsets, null, grad_null):
        leaves = (_leaf(logit), _leaf(env), _leaf(null))
        alpha, null_alpha = kernels.segment_softmax(leaves[0], leaves[1], _dev(offsets), leaves[2])
        g_logit, g_env, g_null = torch.autograd.grad((alpha, null_alpha), leaves, (_dev(grad_alpha), _dev(grad_null)))
        return g_logit.cpu(), g_env.cpu(), g_null.cpu()

    check_segment_softmax_backward(backward)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_force_assembly_golden(dtype):
    announce("golden force_assembly", dtype)

    def run(g, v, src, dst, dst_offsets, src_offsets):
        force, virial = kernels.force_assembly(_dev(g.to(dtype)), _dev(v.to(dtype)), _dev(src), _dev(dst),
                                               _dev(dst_offsets))
        return force.cpu(), virial.cpu()

    check_force(run)


def test_gie_and_rmsnorm_golden():
    announce("golden gie + rmsnorm")
    check_gie(lambda z, r, d, s, i: kernels.zonal_scatter(_dev(z), _dev(r), _dev(d), _dev(s), _dev(i)).cpu())
    check_rmsnorm(lambda x, s, eps: kernels.rmsnorm(_dev(x), _dev(s), eps).cpu())
