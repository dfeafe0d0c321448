"""The allocation-free RMSNorm backward (dpa4k_rmsnorm_backward_noalloc) through the C ABI.

It must give what dpa4k_rmsnorm_backward gives with a caller workspace, bit
for bit (same kernels, same partial order), on consecutive calls that reuse
the library's static scratch array -- each later call smaller than the one
before, so a stale partial row would show -- and both must meet the fp32
rule against the fp64 closed form.
"""
from __future__ import annotations

import pytest
import torch

from bysj_amd.kernels import _lib
from closed_forms import rmsnorm_backward_f64
from parity import announce, assert_bitwise, assert_close_scaled

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _inputs(rows, width, seed, offset=0):
    gen = torch.Generator(device=DEV)
    gen.manual_seed(seed)
    # `offset` floats in front misalign the rows (the element-wise kernels then run)
    x = torch.randn(rows * width + offset, generator=gen, device=DEV)[offset:].reshape(rows, width)
    grad = torch.randn(rows * width + offset, generator=gen, device=DEV)[offset:].reshape(rows, width)
    scale = torch.rand(width, generator=gen, device=DEV) + 0.5
    inverse_rms = torch.rsqrt(x.square().mean(1) + 1e-6)
    return grad, x, scale, inverse_rms


def _with_workspace(library, grad, x, scale, inverse_rms):
    rows, width = x.shape
    grad_x, grad_scale = torch.empty_like(x), torch.empty_like(scale)
    size = library.dpa4k_rmsnorm_backward_workspace_size(rows, width)
    workspace = torch.empty(max(size, 1), dtype=torch.uint8, device=DEV)
    status = library.dpa4k_rmsnorm_backward(grad.data_ptr(), x.data_ptr(), scale.data_ptr(),
                                            inverse_rms.data_ptr(), grad_x.data_ptr(), grad_scale.data_ptr(),
                                            rows, width, workspace.data_ptr(), size,
                                            torch.cuda.current_stream().cuda_stream)
    _lib.check(status)
    return grad_x, grad_scale


def _without_allocation(library, grad, x, scale, inverse_rms):
    rows, width = x.shape
    grad_x, grad_scale = torch.empty_like(x), torch.empty_like(scale)
    status = library.dpa4k_rmsnorm_backward_noalloc(grad.data_ptr(), x.data_ptr(), scale.data_ptr(),
                                                    inverse_rms.data_ptr(), grad_x.data_ptr(),
                                                    grad_scale.data_ptr(), rows, width,
                                                    torch.cuda.current_stream().cuda_stream)
    _lib.check(status)
    return grad_x, grad_scale


def test_noalloc_backward_matches_the_workspace_entry_point():
    library = _lib.load()
    # largest first: every later call uses fewer partial rows or narrower ones than the one before
    shapes = [(24576, 4096, 0), (24576, 1024, 0), (3000, 1024, 0), (300, 256, 0), (37, 1001, 3), (5, 64, 0)]
    for rows, width, offset in shapes:
        announce("rmsnorm backward noalloc", rows, width, offset)
        grad, x, scale, inverse_rms = _inputs(rows, width, seed=rows + width, offset=offset)
        want_x, want_scale = _with_workspace(library, grad, x, scale, inverse_rms)
        got_x, got_scale = _without_allocation(library, grad, x, scale, inverse_rms)
        assert_bitwise(got_x, want_x, f"grad_x {rows}x{width}")
        assert_bitwise(got_scale, want_scale, f"grad_scale {rows}x{width}")
        again_x, again_scale = _without_allocation(library, grad, x, scale, inverse_rms)
        assert_bitwise(again_scale, got_scale, f"grad_scale {rows}x{width}, second call")
        assert_bitwise(again_x, got_x, f"grad_x {rows}x{width}, second call")
        if rows * width <= 3000 * 1024:
            truth_x, truth_scale = rmsnorm_backward_f64(grad, x, scale, 1e-6)
            assert_close_scaled(got_x, truth_x, what="grad_x vs fp64 closed form")
            assert_close_scaled(got_scale, truth_scale, what="grad_scale vs fp64 closed form")


def test_noalloc_backward_without_scale_gradient_and_empty_rows():
    library = _lib.load()
    announce("rmsnorm backward noalloc: no scale gradient, zero rows")
    grad, x, scale, inverse_rms = _inputs(64, 512, seed=7)
    grad_x = torch.empty_like(x)
    stream = torch.cuda.current_stream().cuda_stream
    _lib.check(library.dpa4k_rmsnorm_backward_noalloc(grad.data_ptr(), x.data_ptr(), scale.data_ptr(),
                                                      inverse_rms.data_ptr(), grad_x.data_ptr(), None, 64, 512,
                                                      stream))
    want_x, _ = _with_workspace(library, grad, x, scale, inverse_rms)
    assert_bitwise(grad_x, want_x, "grad_x without grad_scale")
    grad_scale = torch.full((512,), 7.0, device=DEV)
    _lib.check(library.dpa4k_rmsnorm_backward_noalloc(None, None, scale.data_ptr(), None, None,
                                                      grad_scale.data_ptr(), 0, 512, stream))
    assert int(grad_scale.count_nonzero()) == 0
    assert library.dpa4k_rmsnorm_backward_noalloc(None, None, None, None, None, grad_scale.data_ptr(), 4, 512,
                                                  stream) == _lib.EINVAL
    assert b"scale is omitted" in library.dpa4k_last_error()
