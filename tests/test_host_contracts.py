"""Host (CPU) contracts of the operator API: validation, the device gate, autograd wiring.

Restates the behaviour the reference's host tests fix
(tests/python/test_segment_validation.py, test_gie.py:105-166,
test_rmsnorm.py:107-232, test_native_package.py:25-43):

* ``kernels.__all__`` lists the reference's names in its order;
* malformed inputs raise ``TypeError``/``ValueError`` before the device gate;
* well-formed CPU inputs reach the gate, which raises ``RuntimeError``
  (the gate admits gfx950 only);
* the autograd Functions route through the native module's entry points:
  with the gate lifted and ``_extension`` answering with a fake built from
  the oracle, forward values and every input gradient -- including the
  ``edge_scale`` gradient the reference leaves out -- equal the oracle's
  autograd.  The fake is test scaffolding; the product has no CPU path.
"""
from __future__ import annotations

import gc

import importlib
from types import SimpleNamespace
from unittest.mock import patch

import pytest
import torch

from bysj_amd import kernels
from oracle import gie as gie_ref
from oracle import segment as ref

rms_ref = importlib.import_module("oracle.rmsnorm")
segment_mod = importlib.import_module("bysj_amd.kernels.segment")
gie_mod = importlib.import_module("bysj_amd.kernels.gie")
rms_mod = importlib.import_module("bysj_amd.kernels.rmsnorm")
native_mod = importlib.import_module("bysj_amd.kernels.native")

GATE = "gfx950|GPU"


def _graph():
    return torch.tensor([0, 0, 1, 2, 2]), torch.tensor([0, 2, 3, 5])


def test_public_names_match_the_reference_package():
    assert kernels.__all__ == [
        "force_assembly", "gie_available", "gie_zonal_scatter", "group_by_source", "rmsnorm",
        "rmsnorm_available", "segment_available", "segment_offsets", "segment_softmax", "segment_sum",
        "zonal_scatter",
    ]
    for name in kernels.__all__:
        assert callable(getattr(kernels, name))


# ---------------------------------------------------------------------------
# validators (tests/python/test_segment_validation.py)
# ---------------------------------------------------------------------------

def test_segment_sum_validator():
    dst, offsets = _graph()
    src = torch.randn(5, 4)
    assert segment_mod._validate_segment_sum(src, dst, offsets, None, None, None) == 3
    assert segment_mod._validate_segment_sum(src, dst, offsets, torch.rand(5), torch.rand(3), torch.arange(5)) == 3
    assert segment_mod._validate_segment_sum(src, dst, offsets, None, None, torch.arange(5)) == 3
    with pytest.raises(ValueError):
        segment_mod._validate_segment_sum(torch.randn(4, 4), dst, offsets, None, None, None)
    with pytest.raises(TypeError):
        segment_mod._validate_segment_sum(src.double(), dst, offsets, None, None, None)
    with pytest.raises(TypeError):
        segment_mod._validate_segment_sum(src, dst.int(), offsets, None, None, None)
    with pytest.raises(ValueError):
        segment_mod._validate_segment_sum(src, dst, offsets, None, torch.rand(4), None)
    with pytest.raises(ValueError, match="contiguous"):
        segment_mod._validate_segment_sum(torch.randn(4, 5).t(), dst, offsets, None, None, None)


def test_segment_softmax_and_order_validators():
    _, offsets = _graph()
    assert segment_mod._validate_segment_softmax(torch.randn(5, 6), torch.rand(5), offsets, None, None) == (3, 6)
    assert segment_mod._validate_segment_softmax(torch.randn(5, 6), torch.rand(5), offsets, torch.randn(3, 6),
                                                 torch.arange(5)) == (3, 6)
    with pytest.raises(ValueError):
        segment_mod._validate_segment_softmax(torch.randn(5, 6), torch.rand(5), offsets, torch.randn(2, 6), None)
    with pytest.raises(TypeError):
        segment_mod._validate_order(torch.arange(5, dtype=torch.float32), 5, "probe")
    with pytest.raises(ValueError):
        segment_mod._validate_order(torch.arange(4), 5, "probe")
    assert segment_mod._validate_order(None, 5, "probe") is None


def test_force_assembly_validator_and_fp64_extension():
    dst, dst_offsets = _graph()
    src_offsets = torch.tensor([0, 2, 3, 5])
    order = torch.tensor([1, 4, 3, 0, 2])
    g, v = torch.randn(5, 3), torch.randn(5, 3)
    assert segment_mod._validate_force_assembly(g, v, dst_offsets, src_offsets, order) == 3
    assert segment_mod._validate_force_assembly(g.double(), v.double(), dst_offsets, src_offsets, order) == 3
    with pytest.raises(TypeError):
        segment_mod._validate_force_assembly(g, v.double(), dst_offsets, src_offsets, order)
    with pytest.raises(TypeError):
        segment_mod._validate_force_assembly(g.half(), v.half(), dst_offsets, src_offsets, order)
    with pytest.raises(ValueError):
        segment_mod._validate_force_assembly(g, v, dst_offsets, torch.tensor([0, 5]), order)


def test_cpu_csr_helpers_and_range_errors():
    dst = torch.tensor([0, 0, 2, 2, 2])
    assert kernels.segment_offsets(dst, 3).tolist() == [0, 2, 2, 5]
    order, offsets = kernels.group_by_source(torch.tensor([2, 0, 2, 1, 0]), 3)
    assert order.tolist() == [1, 4, 3, 0, 2] and offsets.tolist() == [0, 2, 3, 5]
    with pytest.raises(ValueError):
        kernels.segment_offsets(torch.tensor([0, 3]), 3)
    with pytest.raises(TypeError):
        kernels.segment_offsets(torch.tensor([0, 1], dtype=torch.int32), 3)
    with pytest.raises(ValueError):
        kernels.group_by_source(torch.tensor([0]), 0)


def test_wellformed_cpu_inputs_reach_the_device_gate():
    dst, offsets = _graph()
    with pytest.raises(RuntimeError, match=GATE):
        kernels.segment_sum(torch.randn(5, 4), dst, offsets)
    with pytest.raises(RuntimeError, match=GATE):
        kernels.segment_softmax(torch.randn(5, 4), torch.rand(5), offsets)
    with pytest.raises(RuntimeError, match=GATE):
        kernels.force_assembly(torch.randn(5, 3), torch.randn(5, 3), torch.tensor([2, 0, 2, 1, 0]), dst, offsets)
    with pytest.raises(RuntimeError, match=GATE):
        kernels.zonal_scatter(torch.randn(4, 3), torch.randn(4, 2, 3), torch.tensor([1, 0, 1, 1]),
                              torch.tensor([0, 0, 1]), torch.rand(2))
    with pytest.raises(RuntimeError, match=GATE):
        kernels.rmsnorm(torch.ones(2, 4))


def test_invalid_inputs_fail_before_the_device_gate():
    with pytest.raises(TypeError, match="zonal must be a tensor"):
        kernels.zonal_scatter(None, torch.ones(4, 2, 3), torch.tensor([1, 0, 1, 1]), torch.tensor([0, 0, 1]),
                              torch.rand(2))
    with pytest.raises(ValueError, match="radial must have shape"):
        kernels.zonal_scatter(torch.ones(4, 3), torch.ones(4, 2), torch.tensor([1, 0, 1, 1]), torch.tensor([0, 0, 1]),
                              torch.rand(2))
    with pytest.raises(TypeError, match="dst and radial_slot must be int64"):
        kernels.zonal_scatter(torch.ones(4, 3), torch.ones(4, 2, 3), torch.tensor([1, 0, 1, 1]).int(),
                              torch.tensor([0, 0, 1]), torch.rand(2))
    with pytest.raises(TypeError, match="input must be a tensor"):
        kernels.rmsnorm(None)
    with pytest.raises(ValueError, match="contiguous"):
        kernels.rmsnorm(torch.ones(3, 5).t())
    with pytest.raises(ValueError, match="scale must have shape"):
        kernels.rmsnorm(torch.ones(2, 4), torch.ones(3))
    for eps in (0, -1, float("inf"), float("nan")):
        with pytest.raises(ValueError, match="eps"):
            kernels.rmsnorm(torch.ones(2, 4), eps=eps)


def test_edge_stream_validation_precedes_the_device_gate():
    from bysj_amd.kernels import edge_stream

    x = torch.randn(6, 4, 8)
    with pytest.raises(RuntimeError, match=GATE):
        edge_stream.edge_stream_combine([(1.0, x), (0.5, x, torch.rand(6, 4, 1))], activation="silu")
    with pytest.raises(TypeError, match="sequence"):
        edge_stream.edge_stream_combine(x)
    with pytest.raises(ValueError, match="1 to 4 terms"):
        edge_stream.edge_stream_combine([])
    with pytest.raises(TypeError, match=r"\(coef, a\)"):
        edge_stream.edge_stream_combine([(1.0,)])
    with pytest.raises(TypeError, match="coefficient must be a real number"):
        edge_stream.edge_stream_combine([("2", x)])
    with pytest.raises(ValueError, match="finite"):
        edge_stream.edge_stream_combine([(float("nan"), x)])
    with pytest.raises(TypeError, match="b must be a tensor"):
        edge_stream.edge_stream_combine([(1.0, x, 3.0)])
    with pytest.raises(TypeError, match="float32"):
        edge_stream.edge_stream_combine([(1.0, x.half())])
    with pytest.raises(ValueError, match="more than three"):
        edge_stream.edge_stream_combine([(1.0, x[None])])
    with pytest.raises(ValueError, match=r"\(edges, rows, channels\)"):
        edge_stream.edge_stream_combine([(1.0, torch.randn(4, 8))])
    with pytest.raises(ValueError, match="do not broadcast"):
        edge_stream.edge_stream_combine([(1.0, x), (1.0, torch.randn(6, 3, 8))])
    with pytest.raises(ValueError, match="activation"):
        edge_stream.edge_stream_combine([(1.0, x)], activation="relu")
    with pytest.raises(ValueError, match="gate_rows"):
        edge_stream.edge_stream_combine([(1.0, x)], activation="gate", gate=x, gate_rows=[0])
    with pytest.raises(TypeError, match="gate tensor"):
        edge_stream.edge_stream_combine([(1.0, x)], activation="gate", gate_rows=[-1, 0, 0, 1])
    with pytest.raises(ValueError, match="belong to the gate activation"):
        edge_stream.edge_stream_combine([(1.0, x)], gate=x)
    with pytest.raises(ValueError, match="contiguous tensor of shape"):
        edge_stream.edge_stream_combine([(1.0, x)], out=torch.empty(6, 4, 9))
    with pytest.raises(RuntimeError, match="inference-only"):
        edge_stream.edge_stream_combine([(1.0, x.clone().requires_grad_())])


def test_native_loader_requires_the_entry_point():
    extension = SimpleNamespace(rmsnorm_forward=object())
    with patch.object(native_mod, "_require_hip_runtime"), patch.object(native_mod, "_LOADED", None), \
            patch.object(native_mod.importlib, "import_module", return_value=extension):
        assert native_mod._extension("rmsnorm_forward") is extension
        with pytest.raises(RuntimeError, match="no 'rmsnorm_backward' entry point"):
            native_mod._extension("rmsnorm_backward")
    with patch.object(native_mod, "_require_hip_runtime"), patch.object(native_mod, "_LOADED", None), \
            patch.object(native_mod.importlib, "import_module", side_effect=ImportError("absent")):
        with pytest.raises(RuntimeError, match="not built"):
            native_mod._extension("rmsnorm_forward")


def test_availability_probes_are_false_without_a_gfx950_device():
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    assert not kernels.segment_available()
    assert not kernels.gie_available()
    assert not kernels.rmsnorm_available()


# ---------------------------------------------------------------------------
# autograd wiring against a fake native module built from the oracle
# ---------------------------------------------------------------------------

class _OracleNative:
    """Answers the native module's entry points with the CPU oracle (test scaffolding only)."""

    @staticmethod
    def _dst(offsets, order, edges):
        counts = offsets[1:] - offsets[:-1]
        grouped = torch.repeat_interleave(torch.arange(counts.numel()), counts)
        if order is None:
            return grouped
        dst = torch.empty(edges, dtype=torch.int64)
        dst[order] = grouped
        return dst

    def segment_sum_forward(self, src, offsets, edge_scale=None, node_scale=None, order=None):
        return ref.segment_sum_reference(src, self._dst(offsets, order, src.shape[0]), offsets, edge_scale, node_scale)

    def segment_sum_backward(self, grad_out, src, dst, offsets, edge_scale=None, node_scale=None,
                             want_node_scale_grad=False, order=None, *, want_edge_scale_grad=False):
        grad_src, grad_edge, grad_node = ref.segment_sum_backward_reference(grad_out, src, dst, offsets, edge_scale,
                                                                            node_scale)
        grad_node = grad_node if want_node_scale_grad else None
        if want_edge_scale_grad:
            return grad_src, grad_node, grad_edge
        return grad_src, grad_node

    def segment_softmax_plan(self, offsets, n_edges, channels):
        return ("plan", n_edges, channels)

    def segment_softmax_forward(self, logit, env, offsets, null_logit=None, order=None, *, plan=None):
        assert plan == ("plan", logit.shape[0], logit.shape[1])
        return ref.segment_softmax_reference(logit, env, self._dst(offsets, order, logit.shape[0]), offsets,
                                             null_logit)

    def segment_softmax_backward(self, alpha, grad_alpha, env, offsets, null_alpha=None, grad_null_alpha=None,
                                 order=None, *, plan=None):
        assert plan == ("plan", alpha.shape[0], alpha.shape[1])
        dst = self._dst(offsets, order, alpha.shape[0])
        expectation = torch.zeros(offsets.numel() - 1, alpha.shape[1]).index_add_(0, dst, alpha * grad_alpha)
        if null_alpha is not None:
            expectation = expectation + null_alpha * grad_null_alpha
        grad_logit = alpha * (grad_alpha - expectation[dst])
        grad_null = null_alpha * (grad_null_alpha - expectation) if null_alpha is not None else None
        grad_env = torch.where(env > 0, grad_logit.sum(1) * 2.0 / env, torch.zeros_like(env))
        return grad_logit, grad_null, grad_env

    def gie_zonal_scatter_forward(self, zonal, radial, dst, radial_slot, inv):
        return gie_ref.zonal_scatter_reference(zonal, radial, dst, radial_slot, inv)

    def gie_group(self, dst, radial_slot, n_nodes, n_radial):
        order, offsets = ref.group_by_source(dst, n_nodes)
        return offsets, order, 0

    def gie_zonal_scatter_forward_csr(self, zonal, radial, offsets, order, radial_slot, inv, slot_info=0):
        return gie_ref.zonal_scatter_reference(zonal, radial, self._dst(offsets, order, zonal.shape[0]), radial_slot,
                                               inv)

    def gie_zonal_scatter_backward_csr(self, grad, zonal, radial, offsets, order, radial_slot, inv, slot_info, *,
                                       need=(True, True, True)):
        return gie_ref.zonal_scatter_backward_reference(grad, zonal, radial, self._dst(offsets, order, zonal.shape[0]),
                                                        radial_slot, inv)

    def gie_rmsnorm_supported(self, n_rows, channels):
        return channels % 4 == 0 and (n_rows + 1) * (channels // 4) <= 512

    def gie_rmsnorm_forward_csr(self, zonal, radial, offsets, order, radial_slot, inv, scale, eps, keep_x=False):
        x = gie_ref.zonal_scatter_reference(zonal, radial, self._dst(offsets, order, zonal.shape[0]), radial_slot,
                                            inv)
        flat = x.reshape(x.shape[0], -1)
        y = rms_ref.rmsnorm(flat, scale if scale.numel() else None, eps).reshape(x.shape)
        return y, (x if keep_x else None), torch.rsqrt(flat.square().mean(dim=-1) + eps)

    def rmsnorm_forward(self, x, scale, eps):
        weight = scale if scale.numel() else None
        inv = torch.rsqrt(x.square().mean(dim=-1) + eps).reshape(-1)
        return rms_ref.rmsnorm(x, weight, eps), inv

    def rmsnorm_backward(self, grad, x, scale, inverse_rms, want_scale):
        # closed form on the saved inverse RMS (the eps it was computed with is not passed back)
        width = x.shape[-1]
        rows, g = x.reshape(-1, width), grad.reshape(-1, width)
        inv = inverse_rms.reshape(-1, 1)
        u = g * scale if scale.numel() else g
        grad_x = inv * u - rows * inv ** 3 * (rows * u).mean(1, keepdim=True)
        grad_scale = (g * rows * inv).sum(0) if want_scale else x.new_empty((0,))
        return grad_x.reshape(x.shape), grad_scale


@pytest.fixture
def fake_native():
    fake = _OracleNative()
    with patch.object(segment_mod, "require_dcu"), patch.object(segment_mod, "_extension", return_value=fake), \
            patch.object(gie_mod, "require_dcu"), patch.object(gie_mod, "_extension", return_value=fake), \
            patch.object(rms_mod, "require_dcu"), patch.object(rms_mod, "_extension", return_value=fake):
        yield fake


@pytest.mark.parametrize("use_order", [False, True])
def test_segment_sum_autograd_including_edge_scale(fake_native, use_order):
    gen = torch.Generator().manual_seed(0)
    dst_sorted = torch.tensor([0, 0, 1, 2, 2, 2])
    offsets = torch.tensor([0, 2, 3, 6])
    if use_order:
        perm = torch.tensor([3, 0, 5, 1, 4, 2])
        dst = dst_sorted[perm]
        order, _ = ref.group_by_source(dst, 3)
    else:
        dst, order = dst_sorted, None
    src = torch.randn(6, 4, generator=gen, requires_grad=True)
    w = (torch.rand(6, generator=gen) + 0.5).requires_grad_(True)
    s = (torch.rand(3, 1, generator=gen) + 0.5).requires_grad_(True)
    out = kernels.segment_sum(src, dst, offsets, w, s, order=order)
    expected = ref.segment_sum_reference(src, dst, offsets, w, s.reshape(-1))
    torch.testing.assert_close(out, expected)
    g = torch.randn(out.shape, generator=gen)
    got = torch.autograd.grad(out, (src, w, s), g)
    want = torch.autograd.grad(expected, (src, w, s), g)
    for a, b in zip(got, want):
        torch.testing.assert_close(a, b)
    assert got[2].shape == s.shape


@pytest.mark.parametrize("with_null", [False, True])
def test_segment_softmax_autograd(fake_native, with_null):
    gen = torch.Generator().manual_seed(1)
    dst, offsets = torch.tensor([0, 0, 1, 2, 2, 2]), torch.tensor([0, 2, 3, 6])
    logit = torch.randn(6, 3, generator=gen, requires_grad=True)
    env = (torch.rand(6, generator=gen) + 0.1).requires_grad_(True)
    null = torch.randn(3, 3, generator=gen, requires_grad=True) if with_null else None
    result = kernels.segment_softmax(logit, env, offsets, null)
    expected = ref.segment_softmax_reference(logit, env, dst, offsets, null)
    inputs = (logit, env) + ((null,) if with_null else ())
    if with_null:
        alpha, null_alpha = result
        torch.testing.assert_close(alpha, expected[0])
        torch.testing.assert_close(null_alpha, expected[1])
        cot = (torch.randn(alpha.shape, generator=gen), torch.randn(null_alpha.shape, generator=gen))
        got = torch.autograd.grad(result, inputs, cot)
        want = torch.autograd.grad(expected, inputs, cot)
    else:
        torch.testing.assert_close(result, expected[0])
        cot = torch.randn(result.shape, generator=gen)
        got = torch.autograd.grad(result, inputs, cot)
        want = torch.autograd.grad(expected[0], inputs, cot)
    for a, b in zip(got, want):
        torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-6)


def test_gie_and_rmsnorm_autograd(fake_native):
    gen = torch.Generator().manual_seed(2)
    zonal = torch.randn(4, 3, generator=gen, requires_grad=True)
    radial = torch.randn(4, 2, 3, generator=gen, requires_grad=True)
    dst, slots = torch.tensor([1, 0, 1, 1]), torch.tensor([0, 0, 1])
    inv = (torch.rand(2, generator=gen) + 0.5).requires_grad_(True)
    out = kernels.zonal_scatter(zonal, radial, dst, slots, inv)
    expected = gie_ref.zonal_scatter_reference(zonal, radial, dst, slots, inv)
    torch.testing.assert_close(out, expected)
    g = torch.randn(out.shape, generator=gen)
    for a, b in zip(torch.autograd.grad(out, (zonal, radial, inv), g),
                    torch.autograd.grad(expected, (zonal, radial, inv), g)):
        torch.testing.assert_close(a, b)

    x = torch.randn(2, 3, 11, generator=gen, requires_grad=True)
    scale = torch.randn(11, generator=gen, requires_grad=True)
    out = kernels.rmsnorm(x, scale, eps=1e-5)
    expected = rms_ref.rmsnorm(x, scale, 1e-5)
    torch.testing.assert_close(out, expected)
    g = torch.randn(out.shape, generator=gen)
    for a, b in zip(torch.autograd.grad(out, (x, scale), g), torch.autograd.grad(expected, (x, scale), g)):
        torch.testing.assert_close(a, b)
    out = kernels.rmsnorm(x)
    torch.testing.assert_close(out, rms_ref.rmsnorm(x))


def test_untracked_calls_match_the_autograd_path(fake_native):
    """Without a gradient to record, the operators run their forwards directly: same values, no graph."""
    gen = torch.Generator().manual_seed(5)
    dst, offsets = torch.tensor([0, 0, 1, 2, 2, 2]), torch.tensor([0, 2, 3, 6])
    src = torch.randn(6, 4, generator=gen)
    logit, env = torch.randn(6, 3, generator=gen), torch.rand(6, generator=gen) + 0.1
    null = torch.randn(3, 3, generator=gen)
    x, scale = torch.randn(4, 8, generator=gen), torch.rand(8, generator=gen) + 0.5
    zonal, radial = torch.randn(6, 3, generator=gen), torch.randn(6, 2, 4, generator=gen)
    slots, inv = torch.tensor([0, 1, 1]), torch.rand(3, generator=gen) + 0.5
    rows_scale = torch.rand(16, generator=gen) + 0.5
    calls = {
        "segment_sum": lambda t: kernels.segment_sum(t(src), dst, offsets),
        "segment_softmax": lambda t: kernels.segment_softmax(t(logit), env, offsets, null)[0],
        "rmsnorm": lambda t: kernels.rmsnorm(t(x), scale),
        "zonal_scatter": lambda t: kernels.zonal_scatter(t(zonal), radial, dst, slots, inv),
        "gie_rmsnorm": lambda t: gie_mod.gie_zonal_scatter_rmsnorm(t(zonal), radial, dst, slots, inv, rows_scale),
    }
    for name, call in calls.items():
        tracked = call(lambda v: v.clone().requires_grad_(True))
        assert tracked.grad_fn is not None, name
        plain = call(lambda v: v)
        assert plain.grad_fn is None and not plain.requires_grad, name
        with torch.no_grad():
            quiet = call(lambda v: v.clone().requires_grad_(True))
        assert quiet.grad_fn is None, name
        torch.testing.assert_close(plain, tracked.detach(), rtol=0, atol=0, msg=name)
        torch.testing.assert_close(quiet, tracked.detach(), rtol=0, atol=0, msg=name)


def test_gie_grouping_is_cached_per_dst(fake_native):
    """One grouping per live dst object; in-place writes, new slot tensors and freeing invalidate it."""
    calls = []
    group = fake_native.gie_group

    def counting(*args):
        calls.append(args[2])
        return group(*args)

    fake_native.gie_group = counting
    gie_mod._GROUPINGS.clear()
    gen = torch.Generator().manual_seed(4)
    zonal, radial = torch.randn(5, 3, generator=gen), torch.randn(5, 2, 4, generator=gen)
    dst, slots = torch.tensor([2, 0, 1, 2, 0]), torch.tensor([0, 1, 1])
    inv = torch.rand(3, generator=gen) + 0.5
    first = kernels.zonal_scatter(zonal, radial, dst, slots, inv)
    again = kernels.zonal_scatter(zonal, radial, dst, slots, inv)
    assert len(calls) == 1
    torch.testing.assert_close(again, first)
    gie_mod.gie_zonal_scatter_rmsnorm(zonal, radial, dst, slots, inv)
    assert len(calls) == 1, "the fused operator shares the cache"
    dst.copy_(torch.tensor([0, 0, 1, 2, 2]))  # in place: the version counter moves
    moved = kernels.zonal_scatter(zonal, radial, dst, slots, inv)
    assert len(calls) == 2
    torch.testing.assert_close(moved, gie_ref.zonal_scatter_reference(zonal, radial, dst, slots, inv))
    kernels.zonal_scatter(zonal, radial, dst, slots.clone(), inv)
    assert len(calls) == 3, "another radial_slot object is grouped again"
    kernels.zonal_scatter(zonal, radial, dst, slots, torch.rand(4, generator=gen))
    assert len(calls) == 4, "another node count is grouped again"
    assert len(gie_mod._GROUPINGS) == 1
    gie_mod.require_dcu.reset_mock()  # the stand-in gate keeps its call arguments
    del dst
    gc.collect()
    assert len(gie_mod._GROUPINGS) == 0, "freeing dst drops its entry"


def test_inference_tensors_are_not_cached(fake_native):
    """Tensors made under torch.inference_mode keep no version counter, so no cache can see their
    in-place writes: the softmax runs without a degree plan (the kernels give the same results
    either way) and the GIE grouping is built on every call."""
    plans, groupings = [], []
    fake_native.segment_softmax_plan = lambda *args: plans.append(args)

    def forward_without_plan(logit, env, offsets, null_logit=None, order=None, *, plan=None):
        assert plan is None
        dst = fake_native._dst(offsets, order, logit.shape[0])
        return ref.segment_softmax_reference(logit, env, dst, offsets, null_logit)

    fake_native.segment_softmax_forward = forward_without_plan
    group = fake_native.gie_group
    fake_native.gie_group = lambda *args: groupings.append(args) or group(*args)
    segment_mod._PLANS.clear()
    gie_mod._GROUPINGS.clear()
    gen = torch.Generator().manual_seed(6)
    with torch.inference_mode():
        dst = torch.tensor([0, 0, 1, 2, 2])
        offsets = torch.tensor([0, 2, 3, 5])
        logit, env = torch.randn(5, 4, generator=gen), torch.rand(5, generator=gen) + 0.1
        for _ in range(2):
            alpha = kernels.segment_softmax(logit, env, offsets)
        expected, _ = ref.segment_softmax_reference(logit, env, dst, offsets)
        zonal, radial = torch.randn(5, 3, generator=gen), torch.randn(5, 2, 4, generator=gen)
        slots, inv = torch.tensor([0, 1, 1]), torch.rand(3, generator=gen) + 0.5
        for _ in range(2):
            out = kernels.zonal_scatter(zonal, radial, dst, slots, inv)
        expected_gie = gie_ref.zonal_scatter_reference(zonal, radial, dst, slots, inv)
    torch.testing.assert_close(alpha, expected)
    torch.testing.assert_close(out, expected_gie)
    assert plans == [] and len(segment_mod._PLANS._entries) == 0
    assert len(groupings) == 2 and len(gie_mod._GROUPINGS) == 0


def test_gie_grouping_is_not_built_under_graph_capture(fake_native):
    """Grouping synchronises: under capture only a cached one is used, else a clear error."""
    gie_mod._GROUPINGS.clear()
    zonal, radial = torch.rand(3, 1), torch.rand(3, 1, 4)
    dst, slots, inv = torch.tensor([1, 0, 1]), torch.tensor([0]), torch.rand(2)
    with patch.object(gie_mod, "_capturing", return_value=True):
        with pytest.raises(RuntimeError, match="before HIP graph capture"):
            kernels.zonal_scatter(zonal, radial, dst, slots, inv)
    eager = kernels.zonal_scatter(zonal, radial, dst, slots, inv)
    with patch.object(gie_mod, "_capturing", return_value=True):
        torch.testing.assert_close(kernels.zonal_scatter(zonal, radial, dst, slots, inv), eager)


@pytest.mark.parametrize("with_scale", [False, True])
def test_fused_gie_rmsnorm_autograd(fake_native, with_scale):
    """The fused GIE -> RMSNorm Function: forward and every gradient equal the two operators' chain."""
    gen = torch.Generator().manual_seed(3)
    zonal = torch.randn(6, 3, generator=gen, requires_grad=True)
    radial = torch.randn(6, 2, 4, generator=gen, requires_grad=True)
    dst, slots = torch.tensor([2, 0, 1, 2, 2, 0]), torch.tensor([0, 1, 1])
    inv = (torch.rand(3, generator=gen) + 0.5).requires_grad_(True)
    scale = (torch.rand(16, generator=gen) + 0.5).requires_grad_(True) if with_scale else None
    out = gie_mod.gie_zonal_scatter_rmsnorm(zonal, radial, dst, slots, inv, scale=scale, eps=1e-5)
    rows = gie_ref.zonal_scatter_reference(zonal, radial, dst, slots, inv)
    expected = rms_ref.rmsnorm(rows.reshape(3, 16), scale, 1e-5).reshape(rows.shape)
    torch.testing.assert_close(out, expected)
    inputs = (zonal, radial, inv) + ((scale,) if with_scale else ())
    g = torch.randn(out.shape, generator=gen)
    for a, b in zip(torch.autograd.grad(out, inputs, g), torch.autograd.grad(expected, inputs, g)):
        torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-6)
    with torch.no_grad():  # no gradient wanted: the pre-norm rows are not kept
        assert gie_mod.gie_zonal_scatter_rmsnorm(zonal, radial, dst, slots, inv, scale=scale, eps=1e-5).shape \
            == rows.shape
