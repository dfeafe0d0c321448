"""Host tests of the DeepMD seam layer (bysj_amd/model) -- no GPU, no DeepMD.

Restates the behaviours fixed by the reference's tests/python/test_fused_deepmd.py
and test_dpa4_model.py: each seam against DeepMD's stock path, the fallback
rules and counters, install/uninstall bookkeeping, DeepPot wrapper
resolution, the module dump, the ``fused=`` switch and the facade lifecycle.
Plus what this build adds: the envelope seam's gradient reaches ``edge_env``
(and the source gate), and the CSR view cache cannot serve a stale entry.
"""
from __future__ import annotations

import contextlib
import io
from types import SimpleNamespace
from unittest import mock

import numpy as np
import pytest
import torch

from bysj_amd.model import dpa4, fused_deepmd
from bysj_amd.model.dpa4 import DPA4Model, _normalize_fused
from seam_fakes import (FakeBlock, FakeEdgeCache, FakeModel, OracleOps, edge_force_virial_call, force_namespace,
                        grouped_dst, softmax_namespace)


@pytest.fixture
def any_device():
    fused_deepmd._ACCEPT_ANY_DEVICE = True
    yield
    fused_deepmd.uninstall()
    fused_deepmd._ACCEPT_ANY_DEVICE = False


def _softmax_inputs(seed=0):
    gen = torch.Generator().manual_seed(seed)
    dst = grouped_dst([2, 0, 3, 4])
    logits = torch.randn(9, 2, 3, generator=gen)
    env = torch.rand(9, 1, generator=gen) + 0.1
    env[4] = -1.0
    bias = torch.randn(2, 3, generator=gen)
    return logits, env, dst, 4, bias, 1e-6


# ---------------------------------------------------------------------------
# S1: softmax seam
# ---------------------------------------------------------------------------

def test_softmax_seam_matches_the_stock_path(any_device):
    space, ops = softmax_namespace(), OracleOps()
    stats = fused_deepmd.deepmd_patch(FakeModel([]), ops=ops, namespaces=[space], envelope=False, verbose=False)
    assert stats.bound_softmax
    args = _softmax_inputs()
    actual = space.segment_envelope_gated_softmax(*args)
    fused_deepmd.uninstall()
    expected = space.segment_envelope_gated_softmax(*args)
    torch.testing.assert_close(actual, expected, rtol=2e-5, atol=2e-6)
    assert stats.softmax_hits == 1 and stats.softmax_fallbacks == 0
    assert ops.calls == [("softmax", (9, 6))]


def test_softmax_seam_falls_back_on_source_gating_and_unusable_inputs(any_device):
    space, ops = softmax_namespace(), OracleOps()
    stats = fused_deepmd.deepmd_patch(FakeModel([]), ops=ops, namespaces=[space], envelope=False, verbose=False)
    logits, env, dst, n, bias, eps = _softmax_inputs()
    space.segment_envelope_gated_softmax(logits, env, dst, n, bias, eps, torch.rand(9, 1))  # src_weight
    space.segment_envelope_gated_softmax(logits.double(), env.double(), dst, n, bias.double(), eps)
    # unusable inputs go to the stock path, whatever that path then makes of them
    with contextlib.suppress(RuntimeError):
        space.segment_envelope_gated_softmax(logits, env, dst.int(), n, bias, eps)
    with contextlib.suppress(RuntimeError):
        space.segment_envelope_gated_softmax(logits, env, dst, n, torch.randn(5), eps)
    assert stats.softmax_fallbacks == 4 and stats.softmax_hits == 0 and ops.calls == []


def test_softmax_seam_survives_an_operator_error_and_warns_once(any_device):
    class Broken(OracleOps):
        def segment_softmax(self, *args, **kwargs):
            raise RuntimeError("device lost")

    space = softmax_namespace()
    stats = fused_deepmd.deepmd_patch(FakeModel([]), ops=Broken(), namespaces=[space], envelope=False, verbose=False)
    args = _softmax_inputs()
    with pytest.warns(RuntimeWarning, match="device lost"):
        out = space.segment_envelope_gated_softmax(*args)
    space.segment_envelope_gated_softmax(*args)  # second failure: no second warning required
    assert stats.softmax_fallbacks == 2 and "device lost" in stats.last_error
    fused_deepmd.uninstall()
    torch.testing.assert_close(out, space.segment_envelope_gated_softmax(*args))


def test_softmax_seam_accepts_a_plain_tensor_return(any_device):
    class TensorOps(OracleOps):
        def segment_softmax(self, logit, env, offsets, null_logit=None, *, order=None):
            return OracleOps.segment_softmax(self, logit, env, offsets, null_logit, order=order)[0]

    space = softmax_namespace()
    fused_deepmd.deepmd_patch(FakeModel([]), ops=TensorOps(), namespaces=[space], envelope=False, verbose=False)
    assert tuple(space.segment_envelope_gated_softmax(*_softmax_inputs()).shape) == (9, 2, 3)


# ---------------------------------------------------------------------------
# S2: envelope seam
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("gate", [False, True])
def test_envelope_seam_matches_the_stock_aggregation(any_device, gate):
    cache = FakeEdgeCache([2, 1, 0, 3], gate=gate)
    block = FakeBlock(torch.randn(int(cache.dst.numel()), 2, 4, generator=torch.Generator().manual_seed(3)))
    ops = OracleOps()
    stats = fused_deepmd.deepmd_patch(FakeModel([block]), ops=ops, softmax=False, verbose=False)
    assert stats.bound_envelope and stats.blocks == 1
    x = torch.randn(4, 2, 4)
    actual = block.forward_envelope(x, cache, None)
    fused_deepmd.uninstall()
    expected = block.forward_envelope(x, cache, None)
    torch.testing.assert_close(actual, expected, rtol=1e-5, atol=1e-5 * float(expected.abs().max()))
    assert stats.envelope_hits == 1 and ops.calls[0][0] == "sum"


def test_envelope_seam_gradient_reaches_the_envelope_and_gate(any_device):
    """The reference's seam drops d out / d edge_scale; here forces see the envelope term."""
    cache = FakeEdgeCache([3, 2, 4], gate=True, seed=4)
    message = torch.randn(9, 2, 3, generator=torch.Generator().manual_seed(5), requires_grad=True)
    cache.edge_env.requires_grad_(True)
    cache.edge_src_gate.requires_grad_(True)
    block = FakeBlock(message)
    fused_deepmd.deepmd_patch(FakeModel([block]), ops=OracleOps(), softmax=False, verbose=False)
    x = torch.randn(3, 2, 3)
    upstream = torch.randn(3, 2, 3, generator=torch.Generator().manual_seed(6))
    leaves = (message, cache.edge_env, cache.edge_src_gate)
    got = torch.autograd.grad(block.forward_envelope(x, cache, None), leaves, upstream)
    fused_deepmd.uninstall()
    want = torch.autograd.grad(block.forward_envelope(x, cache, None), leaves, upstream)
    for a, b in zip(got, want):
        torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-6)


def test_envelope_seam_falls_back_in_training_and_on_bad_shapes(any_device):
    cache = FakeEdgeCache([2, 1])
    block = FakeBlock(torch.randn(3, 2, 4))
    ops = OracleOps()
    stats = fused_deepmd.deepmd_patch(FakeModel([block]), ops=ops, softmax=False, verbose=False)
    block.training = True
    block.forward_envelope(torch.randn(2, 2, 4), cache, None)
    block.training = False
    cache.inv_sqrt_deg = torch.rand(5, 1, 1)
    with contextlib.suppress(RuntimeError):  # unusable shapes go to the stock path
        block.forward_envelope(torch.randn(2, 2, 4), cache, None)
    assert stats.envelope_fallbacks == 2 and stats.envelope_hits == 0 and ops.calls == []


# ---------------------------------------------------------------------------
# installation bookkeeping
# ---------------------------------------------------------------------------

def test_uninstall_restores_every_rebound_name(any_device):
    space = softmax_namespace()
    original = space.segment_envelope_gated_softmax
    block = FakeBlock(torch.randn(3, 2, 4))
    fused_deepmd.deepmd_patch(FakeModel([block]), ops=OracleOps(), namespaces=[space], verbose=False)
    assert space.segment_envelope_gated_softmax is not original and "forward_envelope" in block.__dict__
    fused_deepmd.uninstall()
    assert space.segment_envelope_gated_softmax is original
    assert "forward_envelope" not in block.__dict__
    assert block.forward_envelope.__func__ is FakeBlock.forward_envelope


def test_uninstall_keeps_an_earlier_instance_override(any_device):
    block = FakeBlock(torch.randn(3, 2, 4))
    earlier = lambda x, cache, feat: "earlier"  # noqa: E731
    block.forward_envelope = earlier
    fused_deepmd.deepmd_patch(FakeModel([block]), ops=OracleOps(), softmax=False, verbose=False)
    assert block.forward_envelope is not earlier
    block.training = True  # fallback: the stock callable is the earlier override
    assert block.forward_envelope(torch.randn(2, 2, 4), FakeEdgeCache([2, 1]), None) == "earlier"
    fused_deepmd.uninstall()
    assert block.forward_envelope is earlier


def test_install_is_a_noop_without_the_operators(any_device):
    model = FakeModel([FakeBlock(torch.zeros(2, 1, 1))])
    stats = fused_deepmd.deepmd_patch(model, ops=None, verbose=False)
    if fused_deepmd._segment_operators() is None:  # no gfx950 device here
        assert not (stats.bound_softmax or stats.bound_envelope)
    assert fused_deepmd.status(stats)["blocks"] == 1
    assert fused_deepmd.status(None) == {}


def test_installing_twice_keeps_one_patch(any_device):
    space = softmax_namespace()
    original = space.segment_envelope_gated_softmax
    first = fused_deepmd.deepmd_patch(FakeModel([]), ops=OracleOps(), namespaces=[space], envelope=False,
                                      verbose=False)
    second = fused_deepmd.deepmd_patch(FakeModel([]), ops=OracleOps(), namespaces=[space], envelope=False,
                                       verbose=False)
    assert [k for k in fused_deepmd.installed() if k.endswith(".segment_envelope_gated_softmax")] == [
        "fake.sezm_nn.attention.segment_envelope_gated_softmax"]
    space.segment_envelope_gated_softmax(*_softmax_inputs())
    assert first.softmax_hits == 0 and second.softmax_hits == 1
    fused_deepmd.uninstall()
    assert space.segment_envelope_gated_softmax is original


def test_wrappers_resolve_to_their_module_tree(any_device):
    root = FakeModel([])
    assert fused_deepmd._module_root(SimpleNamespace(deep_eval=SimpleNamespace(dp=root))) == (root, "deep_eval.dp")
    assert fused_deepmd._module_root(SimpleNamespace(deep_eval=SimpleNamespace(_dpmodel=root))) == (
        root, "deep_eval._dpmodel")
    assert fused_deepmd._module_root(SimpleNamespace(deep_eval=SimpleNamespace())) == (None, "")
    assert "no nn.Module tree" in "\n".join(fused_deepmd.describe_module(SimpleNamespace(deep_eval=None)))
    cache = FakeEdgeCache([2, 1, 3])
    block = FakeBlock(torch.randn(6, 2, 4))
    stats = fused_deepmd.deepmd_patch(SimpleNamespace(deep_eval=SimpleNamespace(dp=FakeModel([block]))),
                                      ops=OracleOps(), softmax=False, verbose=False)
    block.forward_envelope(torch.randn(3, 2, 4), cache, None)
    assert stats.blocks == 1 and stats.envelope_hits == 1


def test_module_dump_and_verbose_install():
    block = FakeBlock(torch.randn(3, 2, 4))
    text = "\n".join(fused_deepmd.describe_module(FakeModel([block])))
    assert "module: FakeModel" in text and "patch targets: 1 SO(2) block(s)" in text
    assert "forward_envelope -> segment_sum" in text
    buffer = io.StringIO()
    fused_deepmd._ACCEPT_ANY_DEVICE = True
    try:
        with contextlib.redirect_stdout(buffer):
            fused_deepmd.deepmd_patch(FakeModel([]), ops=OracleOps(), namespaces=[softmax_namespace()],
                                      envelope=False)
    finally:
        fused_deepmd.uninstall()
        fused_deepmd._ACCEPT_ANY_DEVICE = False
    assert "[deepmd_patch] module:" in buffer.getvalue()
    assert "segment_envelope_gated_softmax" in buffer.getvalue()


# ---------------------------------------------------------------------------
# CSR view cache
# ---------------------------------------------------------------------------

def test_csr_view_reuses_and_invalidates_entries():
    view = fused_deepmd._CsrView(capacity=2)
    dst = torch.tensor([2, 0, 2, 1, 0])
    offsets, order = view.get(dst, 3)
    assert offsets.tolist() == [0, 2, 3, 5] and order.tolist() == [1, 4, 3, 0, 2]
    again = view.get(dst, 3)
    assert again[0] is offsets and again[1] is order          # cached
    dst[0] = 1                                                  # in-place write moves the version counter
    fresh_offsets, _ = view.get(dst, 3)
    assert fresh_offsets is not offsets and fresh_offsets.tolist() == [0, 2, 4, 5]
    assert view.get(dst, 4)[0].tolist() == [0, 2, 4, 5, 5]      # another node count is another view
    others = [torch.tensor([0, 1]) for _ in range(3)]
    for other in others:
        view.get(other, 2)
    assert len(view) == 2                                       # LRU capacity
    del others, other
    assert len(view) == 0                                       # freed tensors drop their entries


def test_csr_view_leaves_sorted_destinations_in_natural_order():
    """A non-decreasing dst needs no order: the operators then take their natural-order kernels."""
    view = fused_deepmd._CsrView()
    offsets, order = view.get(torch.tensor([0, 0, 1, 2, 2]), 3)
    assert order is None and offsets.tolist() == [0, 2, 3, 5]
    with pytest.raises(ValueError, match="node range"):
        view.get(torch.tensor([0, 3]), 3)


def test_csr_view_of_inference_tensors_is_built_per_call():
    """Inference tensors keep no version counter, so their views are not kept (and do not raise)."""
    view = fused_deepmd._CsrView()
    with torch.inference_mode():
        dst = torch.tensor([1, 0, 1, 2])
        offsets, order = view.get(dst, 3)
        again = view.get(dst, 3)
    assert offsets.tolist() == [0, 1, 3, 4] and order.tolist() == [1, 0, 2, 3]
    assert again[0].tolist() == offsets.tolist() and len(view) == 0


# ---------------------------------------------------------------------------
# fused= switch and DPA4Model facade
# ---------------------------------------------------------------------------

def test_fused_switch_normalisation():
    assert _normalize_fused(True) == {"softmax": True, "envelope": True}
    assert _normalize_fused("softmax") == {"softmax": True}
    assert _normalize_fused(("envelope",)) == {"envelope": True}
    assert _normalize_fused({"softmax": True, "envelope": False}) == {"softmax": True, "envelope": False}
    for off in (False, None, ()):
        assert _normalize_fused(off) is None
    for bad in ("flash", {"flash": True}):
        with pytest.raises(ValueError):
            _normalize_fused(bad)
    with pytest.raises(TypeError):
        _normalize_fused(3)


class _Backend:
    def __init__(self, module_name):
        self.__class__ = type("Backend", (_Backend,), {"__module__": module_name})


class _FakeDeepPot:
    def __init__(self, backend="deepmd.pt.infer.deep_eval"):
        self.deep_eval = _Backend(backend)
        self.calls, self.closed = [], False

    def eval(self, coords, cells, atom_types, **kwargs):
        self.calls.append((coords, cells, atom_types, kwargs))
        return {"energy": 1.0, "force": 2.0, "virial": 3.0}

    def get_rcut(self):
        return 6.0

    def get_type_map(self):
        return ["O", "H"]

    def get_ntypes(self):
        return 2

    def get_model_def_script(self):
        return {"type": "dpa4"}

    def close(self):
        self.closed = True


def _facade(pot, **kwargs):
    with mock.patch.object(dpa4, "_create_deep_pot", return_value=pot):
        return DPA4Model("water.pt", **kwargs)


def test_facade_forwards_eval_and_queries():
    pot = _FakeDeepPot()
    model = _facade(pot)
    coords, cells, types_ = np.zeros((1, 3, 3)), np.zeros((1, 3, 3)), np.zeros((1, 3), dtype=int)
    assert model.eval(coords, cells, types_, atomic=True, fparam=[0.5], aparam=[0.1])["energy"] == 1.0
    c, ce, t, kwargs = pot.calls[0]
    assert c is coords and ce is cells and t is types_
    assert kwargs == {"atomic": True, "fparam": [0.5], "aparam": [0.1]}
    assert model.predict.__func__ is model.eval.__func__
    assert (model.get_rcut(), model.get_type_map(), model.get_ntypes()) == (6.0, ["O", "H"], 2)
    assert model.get_model_def_script() == {"type": "dpa4"}
    assert _facade(_FakeDeepPot("deepmd.pt_expt.infer.deep_eval")).backend == "pt_expt"
    assert _facade(_FakeDeepPot("torch")).backend == "unknown"
    assert model.backend == "pt"


def test_facade_installs_the_seams_and_uninstalls_once():
    pot = _FakeDeepPot()
    report = {"softmax_hits": 0, "bound_softmax": True}
    with mock.patch.object(dpa4, "_create_deep_pot", return_value=pot), \
            mock.patch.object(fused_deepmd, "deepmd_patch") as patch, \
            mock.patch.object(fused_deepmd, "status", return_value=report), \
            mock.patch.object(fused_deepmd, "uninstall") as uninstall:
        model = DPA4Model("water.pt", fused=True)
        patch.assert_called_once_with(pot, softmax=True, envelope=True, force=False)
        assert model.fused_ops == report and model.fused_seams == {"softmax": True, "envelope": True}
        assert "fused_ops={'softmax_hits': 0" in repr(model)
        model.close()
        model.close()
        uninstall.assert_called_once_with(pot)
        assert pot.closed and model.fused_ops == {}
        with DPA4Model("water.pt", fused=("softmax",)) as scoped:
            assert isinstance(scoped, DPA4Model)
    assert pot.closed


@pytest.mark.parametrize("fused, switches", [
    (("force",), {"softmax": False, "envelope": False, "force": True}),
    ("envelope", {"softmax": False, "envelope": True, "force": False}),
    ({"softmax": True}, {"softmax": True, "envelope": False, "force": False}),
    ({"envelope": False, "force": True}, {"softmax": False, "envelope": False, "force": True}),
])
def test_facade_switches_off_every_seam_it_does_not_select(fused, switches):
    """deepmd_patch turns the reference's two seams on by default: a partial selection passes every switch."""
    with mock.patch.object(dpa4, "_create_deep_pot", return_value=_FakeDeepPot()), \
            mock.patch.object(fused_deepmd, "deepmd_patch") as patch, \
            mock.patch.object(fused_deepmd, "status", return_value={"x": 1}):
        DPA4Model("water.pt", fused=fused)
    assert patch.call_args.kwargs == switches


def test_any_false_switch_installs_nothing():
    for off in (False, None, (), 0, "", [], {}, np.bool_(False)):
        assert _normalize_fused(off) is None, off
    with mock.patch.object(dpa4, "_create_deep_pot", return_value=_FakeDeepPot()), \
            mock.patch.object(fused_deepmd, "deepmd_patch") as patch:
        DPA4Model("water.pt", fused=0)
    patch.assert_not_called()


def test_facade_rejects_bad_switches_before_loading():
    with mock.patch.object(dpa4, "_create_deep_pot") as create:
        with pytest.raises(ValueError, match="unknown fused seam"):
            DPA4Model("water.pt", fused="flash")
        for keyword in ("tilelang_ops", "native_ops"):
            with pytest.raises(RuntimeError, match=f"{keyword} was removed"):
                DPA4Model("water.pt", **{keyword: ("gie",)})
    create.assert_not_called()
    with mock.patch.object(fused_deepmd, "deepmd_patch") as patch:
        assert _facade(_FakeDeepPot()).fused_ops == {}
    patch.assert_not_called()


def test_facade_without_deepmd_says_so():
    with pytest.raises(RuntimeError, match="DeepMD-kit"):
        DPA4Model("water.pt")


# ---------------------------------------------------------------------------
# S3: force seam (opt-in)
# ---------------------------------------------------------------------------

def _force_case(n_ext=7, n_edges=40, seed=3, dtype=torch.float32):
    gen = torch.Generator().manual_seed(seed)
    dst = torch.randint(0, n_ext, (n_edges,), generator=gen)  # unsorted, as DeepMD's extended lists are
    src = torch.randint(0, n_ext, (n_edges,), generator=gen)
    g = torch.randn(n_edges, 3, generator=gen, dtype=torch.float64).to(dtype)
    vec = torch.randn(n_edges, 3, generator=gen, dtype=torch.float64).to(dtype)
    return g, vec, dst, src, n_ext


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_force_seam_matches_the_stock_chain(any_device, dtype):
    g, vec, dst, src, n_ext = _force_case(dtype=dtype)
    space, ops = force_namespace(), OracleOps()
    stats = fused_deepmd.deepmd_patch(FakeModel([]), ops=ops, softmax=False, envelope=False, force=True,
                                      force_namespaces=[(space, "edge_force_virial")], verbose=False)
    assert stats.bound_force and fused_deepmd.installed() == ["fake.pt_expt.kernels.edge_force_virial.edge_force_virial"]
    args = edge_force_virial_call(g, vec, dst, src, n_ext)
    force, atom_virial, frame_virial, extra = space.edge_force_virial(*args)
    fused_deepmd.uninstall()
    assert space.edge_force_virial.__name__ == "stock_edge_force_virial"
    e_force, e_atom, e_frame, _ = space.edge_force_virial(*args)
    tolerance = dict(rtol=1e-12, atol=1e-12) if dtype == torch.float64 else dict(rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(force, e_force, **tolerance)
    torch.testing.assert_close(atom_virial, e_atom, **tolerance)
    torch.testing.assert_close(frame_virial, e_frame, **tolerance)
    assert extra is None and force.shape == (3 * n_ext,) and frame_virial.shape == (1, 9)
    assert stats.force_hits == 1 and stats.force_fallbacks == 0 and ops.calls == [("force", (40, 3))]


@pytest.mark.parametrize("case", ["masked_edge", "two_frames", "optional_tensor", "wrong_dtype", "bad_row_ptr"])
def test_force_seam_falls_back_where_the_quote_is_silent(any_device, case):
    g, vec, dst, src, n_ext = _force_case(n_ext=8)
    kwargs = {}
    if case == "masked_edge":
        mask = torch.ones(g.shape[0], dtype=torch.bool)
        mask[5] = False
        kwargs["edge_mask"] = mask
    elif case == "two_frames":
        kwargs["frames"] = 2
    elif case == "optional_tensor":
        kwargs["optional"] = torch.ones(3)
    args = list(edge_force_virial_call(g, vec, dst, src, n_ext, **kwargs))
    if case == "wrong_dtype":
        args[0], args[1] = args[0].half(), args[1].half()
    if case == "bad_row_ptr":
        args[5] = args[5][:-1]
    space, ops = force_namespace(), OracleOps()
    stats = fused_deepmd.deepmd_patch(FakeModel([]), ops=ops, softmax=False, envelope=False, force=True,
                                      force_namespaces=[(space, "edge_force_virial")], verbose=False)
    if case not in ("wrong_dtype", "bad_row_ptr"):
        result = space.edge_force_virial(*args)
        torch.testing.assert_close(result[0], force_namespace().edge_force_virial(*args)[0])
    else:
        try:
            space.edge_force_virial(*args)
        except (RuntimeError, IndexError):  # the stock chain itself rejects these inputs
            pass
    assert stats.force_hits == 0 and stats.force_fallbacks == 1 and ops.calls == []


def test_force_seam_is_opt_in_and_reports_missing_homes(any_device):
    space = force_namespace()
    stats = fused_deepmd.deepmd_patch(FakeModel([]), ops=OracleOps(), softmax=False, envelope=False,
                                      force_namespaces=[(space, "edge_force_virial")], verbose=False)
    assert not stats.bound_force and fused_deepmd.installed() == []
    assert _normalize_fused(True) == {"softmax": True, "envelope": True}
    assert _normalize_fused(("force",)) == {"force": True}
    buffer = io.StringIO()
    with contextlib.redirect_stdout(buffer):
        stats = fused_deepmd.deepmd_patch(FakeModel([]), ops=OracleOps(), softmax=False, envelope=False,
                                          force=True, force_namespaces=[])
    assert not stats.bound_force and "edge_force_virial is not importable here" in buffer.getvalue()
    fused_deepmd.uninstall()


def test_force_seam_derives_its_slot_order_once_per_grouping_pair(any_device):
    """The same (dst_order, src_order) objects give the operator the same slot_order object (so its plan cache
    hits); an in-place write to either grouping or another pair derives it again; an identity dst_order makes
    the seam pass the values without a gather."""
    g, vec, dst, src, n_ext = _force_case(n_ext=9, n_edges=60, seed=8)
    seen = []

    class Recording(OracleOps):
        def force_assembly(self, grad_edge, edge_vec, src, dst, dst_offsets, src_offsets=None, src_order=None):
            seen.append((grad_edge, src_order))
            return super().force_assembly(grad_edge, edge_vec, src, dst, dst_offsets, src_offsets, src_order)

    space = force_namespace()
    fused_deepmd.deepmd_patch(FakeModel([]), ops=Recording(), softmax=False, envelope=False, force=True,
                              force_namespaces=[(space, "edge_force_virial")], verbose=False)
    args = edge_force_virial_call(g, vec, dst, src, n_ext)
    first = space.edge_force_virial(*args)
    second = space.edge_force_virial(*args)
    assert seen[0][1] is seen[1][1], "the slot order is derived once per grouping pair"
    torch.testing.assert_close(first[0], second[0], rtol=0, atol=0)
    args[6].add_(0)  # an in-place write to src_order: derived again
    space.edge_force_virial(*args)
    assert seen[2][1] is not seen[1][1]
    torch.testing.assert_close(seen[2][1], seen[1][1], rtol=0, atol=0)
    # destination-sorted natural order: dst_order is the identity and the values go in as they are
    order = torch.argsort(dst, stable=True)
    sorted_args = list(edge_force_virial_call(g[order].contiguous(), vec[order].contiguous(), dst[order], src[order],
                                              n_ext))
    sorted_args[4] = torch.arange(60)  # a stable grouping of a sorted list (the quoted argsort may swap ties)
    result = space.edge_force_virial(*sorted_args)
    assert seen[-1][0] is sorted_args[0]
    fused_deepmd.uninstall()
    expected = space.edge_force_virial(*sorted_args)
    torch.testing.assert_close(result[0], expected[0], rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(result[1], expected[1], rtol=1e-5, atol=1e-5)
