"""Binds the gfx950 segment operators into a loaded DeepMD DPA4/SeZM model.

The reference's seam layer (python/model/fused_deepmd.py:103-462 of
lipengfei1409/bysj) rebinds two of DeepMD's own dispatch points; this module
offers the same public surface (``deepmd_patch``, ``uninstall``, ``status``,
``describe_module``, ``FusedStats``) over this build's operators, plus a third
seam.  DeepMD itself is never edited, and every seam keeps DeepMD's own
implementation as its fallback:

softmax   ``segment_envelope_gated_softmax(logits, edge_env, dst, n_nodes,
          z_bias_raw, eps, src_weight=None)``, the eager softmax that
          ``SO2Convolution.attention_weights`` calls.  Served by
          ``segment_softmax`` with the null logit ``log(softplus(z_bias) +
          eps)``; the envelope is folded into the logit inside the kernel.

envelope  ``SO2Convolution.forward_envelope(self, x, edge_cache,
          radial_feat)``, the attention-free aggregation ``zeros ->
          index_add_(dst) -> mul_``.  Served by one ``segment_sum`` with
          ``edge_scale = edge_env * edge_src_gate`` and ``node_scale =
          inv_sqrt_deg``; the gradient reaches ``edge_scale`` (DeepMD's
          envelope depends on the coordinates, so forces need it).

force     ``edge_force_virial`` (module ``deepmd.pt_expt.kernels.
          edge_force_virial``; ``transform_output`` imports it as
          ``fused_edge_force_virial``), the per-atom force and virial from the
          per-edge energy gradients (call quoted at docs/fused-operators.md:
          117-130 of the reference, which leaves it unwired).  Served by
          ``force_assembly`` for one frame with no masked edges and an empty
          optional tensor; everything else goes to DeepMD's function.  Opt-in:
          ``deepmd_patch(..., force=True)``.

The destination CSR of ``dst`` is built once per neighbour graph on the device
and cached per ``dst`` tensor object (:class:`_CsrView`).  :class:`FusedStats`
counts hits and fallbacks; a seam falls back when its inputs are outside what
the kernels take or when the operator raises, and the first error is reported
once as a warning.
"""
from __future__ import annotations

import importlib
import warnings
import weakref
from dataclasses import asdict, dataclass
from types import MethodType
from typing import Any, Callable, Iterable

import torch
import torch.nn.functional as F

# Host tests drive the seams with CPU tensors and a stand-in operator bundle;
# in a real install CPU tensors stay on DeepMD's path.  Only a test sets this.
_ACCEPT_ANY_DEVICE = False

_SOFTMAX_NAME = "segment_envelope_gated_softmax"
_ENVELOPE_NAME = "forward_envelope"
# Where DeepMD keeps each rebound name (modules imported only on a real install).
_SOFTMAX_HOMES = (
    "deepmd.pt.model.descriptor.sezm_nn.attention",
    "deepmd.pt.model.descriptor.sezm_nn.so2",
    "deepmd.pt.model.descriptor.sezm_nn",
)
_FORCE_HOMES = (
    ("deepmd.pt_expt.kernels.edge_force_virial", "edge_force_virial"),
    ("deepmd.pt.model.model.transform_output", "fused_edge_force_virial"),
)
# Attributes of a DeepPot's ``deep_eval`` that hold the torch module tree: the
# legacy ``pt`` backend's ModelWrapper, the ``pt_expt`` backend's
# deserialized graph, a generic ``model``; ``deep_eval`` itself comes last.
_TREE_ATTRIBUTES = ("dp", "_dpmodel", "model")
_CSR_CAPACITY = 4


@dataclass
class FusedStats:
    """Hit, fallback and error counters of one installation."""

    softmax_hits: int = 0
    softmax_fallbacks: int = 0
    envelope_hits: int = 0
    envelope_fallbacks: int = 0
    force_hits: int = 0
    force_fallbacks: int = 0
    bound_softmax: bool = False
    bound_envelope: bool = False
    bound_force: bool = False
    blocks: int = 0
    last_error: str | None = None

    def as_dict(self) -> dict[str, Any]:
        return asdict(self)


# ---------------------------------------------------------------------------
# operands and operators
# ---------------------------------------------------------------------------

def _on_device(tensor: torch.Tensor) -> bool:
    return tensor.is_cuda or _ACCEPT_ANY_DEVICE


def _kernel_operand(value: Any, dtypes=(torch.float32,)) -> bool:
    """A tensor the kernels take: one of ``dtypes``, contiguous, on the GPU."""
    return (isinstance(value, torch.Tensor) and value.dtype in dtypes and value.is_contiguous()
            and _on_device(value))


def _index_operand(value: Any) -> bool:
    return _kernel_operand(value, (torch.int64,)) and value.dim() == 1


def _kernels_segment():
    """This build's ``kernels.segment`` module (ImportError when absent)."""
    try:
        from ..kernels import segment
    except ImportError:  # bysj_amd/ on sys.path: this package imported as the reference's `model`
        from kernels import segment
    return segment


def _segment_operators():
    """``kernels.segment`` when it can run on this host, else None."""
    try:
        segment = _kernels_segment()
    except ImportError:
        return None
    return segment if segment.segment_available() else None


def _destination_grouping(dst: torch.Tensor, n_nodes: int):
    """``(offsets, order)``; ``order`` is None when ``dst`` is already non-decreasing."""
    return _kernels_segment().destination_grouping(dst, n_nodes)


class _CsrView:
    """Destination CSR views ``(offsets, order)`` of recent ``dst`` tensors (LRU).

    Keyed by the identity of the ``dst`` tensor object; an entry is valid
    while that object is alive and its storage, size, version counter and
    node count are unchanged.  An inference tensor keeps no version counter,
    so its view is built on every call and not kept.
    """

    def __init__(self, capacity: int = _CSR_CAPACITY):
        self.capacity = capacity
        self._entries: dict[int, tuple] = {}   # id(dst) -> (weakref, stamp, offsets, order)

    @staticmethod
    def _stamp(dst: torch.Tensor, n_nodes: int):
        if dst.is_inference():
            return None
        return (dst.data_ptr(), dst.numel(), dst._version, str(dst.device), int(n_nodes))

    def get(self, dst: torch.Tensor, n_nodes: int):
        stamp = self._stamp(dst, n_nodes)
        if stamp is None:
            return _destination_grouping(dst, int(n_nodes))
        key = id(dst)
        entry = self._entries.pop(key, None)
        if entry is not None and entry[0]() is dst and entry[1] == stamp:
            self._entries[key] = entry            # most recently used last
            return entry[2], entry[3]
        offsets, order = _destination_grouping(dst, int(n_nodes))
        reference = weakref.ref(dst, lambda _, key=key: self._entries.pop(key, None))
        self._entries[key] = (reference, stamp, offsets, order)
        while len(self._entries) > self.capacity:
            self._entries.pop(next(iter(self._entries)))
        return offsets, order

    def __len__(self) -> int:
        return len(self._entries)


class _ForceView:
    """What the force seam derives from DeepMD's two edge groupings, per ``(dst_order, src_order)`` pair (LRU).

    ``force_assembly`` takes the values in destination order and names each
    source slot's edge by its destination slot: ``slot_order[q] =
    rank[src_order[q]]``, with ``rank`` the inverse of ``dst_order``.  Built
    once per pair of tensor objects (one host synchronisation, to learn
    whether ``dst_order`` is the identity, in which case the values need no
    gather) and kept while both objects live unchanged, so that later calls
    hand the same ``slot_order`` object to the operator, whose blob plan is
    cached per that object.  Inference tensors keep no version counter:
    nothing is kept for them.
    """

    def __init__(self, capacity: int = _CSR_CAPACITY):
        self.capacity = capacity
        self._entries: dict[tuple, tuple] = {}  # key -> (dst ref, src ref, stamps, slot_order, identity)

    @staticmethod
    def _stamp(tensor: torch.Tensor):
        if tensor.is_inference():
            return None
        return (tensor.data_ptr(), tensor.numel(), tensor._version, str(tensor.device))

    @staticmethod
    def _derive(dst_order: torch.Tensor, src_order: torch.Tensor) -> tuple[torch.Tensor, bool]:
        edges = dst_order.numel()
        slots = torch.arange(edges, device=dst_order.device, dtype=dst_order.dtype)
        rank = torch.empty_like(dst_order)
        rank[dst_order] = slots
        identity = bool(torch.equal(dst_order, slots))
        return rank.index_select(0, src_order).contiguous(), identity

    def _forget(self, key: tuple) -> None:
        entry = self._entries.get(key)
        if entry is not None and (entry[0]() is None or entry[1]() is None):
            del self._entries[key]

    def get(self, dst_order: torch.Tensor, src_order: torch.Tensor) -> tuple[torch.Tensor, bool]:
        stamps = (self._stamp(dst_order), self._stamp(src_order))
        if stamps[0] is None or stamps[1] is None:
            return self._derive(dst_order, src_order)
        key = (id(dst_order), id(src_order))
        entry = self._entries.pop(key, None)
        if entry is not None and entry[0]() is dst_order and entry[1]() is src_order and entry[2] == stamps:
            self._entries[key] = entry            # most recently used last
            return entry[3], entry[4]
        slot_order, identity = self._derive(dst_order, src_order)
        forget = lambda _, key=key: self._forget(key)  # noqa: E731
        self._entries[key] = (weakref.ref(dst_order, forget), weakref.ref(src_order, forget), stamps, slot_order,
                              identity)
        while len(self._entries) > self.capacity:
            self._entries.pop(next(iter(self._entries)))
        return slot_order, identity

    def __len__(self) -> int:
        return len(self._entries)


# ---------------------------------------------------------------------------
# finding the seams
# ---------------------------------------------------------------------------

def _module_root(model: Any) -> tuple[Any | None, str]:
    """The ``nn.Module`` tree behind ``model`` and the dotted path it was found at.

    ``model`` itself when it is a module tree (path ``"model"``); otherwise
    the first of ``deep_eval.<attr>`` (see ``_TREE_ATTRIBUTES``) and then
    ``deep_eval`` that has one; ``(None, "")`` when there is none.
    """
    def is_tree(candidate: Any) -> bool:
        return candidate is not None and callable(getattr(candidate, "modules", None))

    if is_tree(model):
        return model, "model"
    evaluator = getattr(model, "deep_eval", None)
    if evaluator is None:
        return None, ""
    paths = [(f"deep_eval.{name}", getattr(evaluator, name, None)) for name in _TREE_ATTRIBUTES]
    paths.append(("deep_eval", evaluator))
    return next(((tree, path) for path, tree in paths if is_tree(tree)), (None, ""))


def _is_so2_block(module: Any) -> bool:
    """A SeZM SO(2) convolution: it carries both aggregation seams."""
    return (hasattr(module, "_segment_softmax_fn") and callable(getattr(module, "edge_message", None))
            and callable(getattr(module, _ENVELOPE_NAME, None)))


def _so2_blocks(root: Any) -> list[Any]:
    return [] if root is None else [module for module in root.modules() if _is_so2_block(module)]


def _importable(names: Iterable[str]) -> list[Any]:
    """The modules of ``names`` that import here (DeepMD is optional)."""
    found = []
    for name in names:
        try:
            found.append(importlib.import_module(name))
        except ImportError:
            continue
    return found


def describe_module(module: Any, *, max_depth: int = 2, max_rows: int = 40) -> list[str]:
    """Printable lines: the module tree down to ``max_depth`` and every patch target."""
    root, path = _module_root(module)
    kind = type(module).__name__
    if root is None:
        return [f"module: {kind} (no nn.Module tree found -- pass an nn.Module, or a DeepPot/DeepEval "
                "wrapper holding one at deep_eval.dp or deep_eval._dpmodel)",
                "patch targets: 0 (nothing can be bound)"]
    rows = list(root.named_modules()) if hasattr(root, "named_modules") else []
    shown = [(name, child) for name, child in rows[:max_rows] if (name.count(".") + 1 if name else 0) <= max_depth]
    suffix = "" if path == "model" else f" -> {path}"
    report = [f"module: {kind}{suffix} ({type(root).__name__}, {len(rows)} submodules)"]
    report += [f"  {'  ' * (name.count('.') + 1 if name else 0)}{name or '<root>'}  {type(child).__name__}"
               for name, child in shown]
    if len(rows) > max_rows:
        report.append(f"  ... {len(rows) - max_rows} more submodules")
    blocks = _so2_blocks(root)
    report.append(f"patch targets: {len(blocks)} SO(2) block(s)")
    report += [f"  [{i}] {type(block).__name__}  n_atten_head={getattr(block, 'n_atten_head', '?')}  "
               "seams: forward_envelope -> segment_sum, attention softmax -> segment_softmax"
               for i, block in enumerate(blocks)]
    return report


# ---------------------------------------------------------------------------
# the installation
# ---------------------------------------------------------------------------

class _Rebinding:
    """One name rebound on an object, and how to put it back.

    For a module attribute the previous value is restored.  For a method
    patched on an instance, the instance's own attribute is restored when it
    had one, else removed, so that the class's method shows through again.
    """

    __slots__ = ("owner", "name", "previous", "on_instance")

    def __init__(self, owner: Any, name: str, value: Any, *, on_instance: bool):
        self.owner, self.name, self.on_instance = owner, name, on_instance
        if on_instance:
            self.previous = vars(owner).get(name)
            vars(owner)[name] = value
        else:
            self.previous = getattr(owner, name)
            setattr(owner, name, value)

    def undo(self) -> None:
        if not self.on_instance:
            setattr(self.owner, self.name, self.previous)
        elif self.previous is None:
            vars(self.owner).pop(self.name, None)
        else:
            vars(self.owner)[self.name] = self.previous

    def label(self) -> str:
        where = getattr(self.owner, "__name__", None) or f"{type(self.owner).__name__}@{id(self.owner):x}"
        return f"{where}.{self.name}"


class _Installation:
    """The operators, counters, CSR cache and rebindings of one ``deepmd_patch``."""

    def __init__(self, ops: Any, stats: FusedStats):
        self.ops, self.stats = ops, stats
        self.csr = _CsrView()
        self.force_views = _ForceView()
        self.rebindings: list[_Rebinding] = []
        self.warned = False

    def rebind(self, owner: Any, name: str, value: Any, *, on_instance: bool = False) -> None:
        self.rebindings.append(_Rebinding(owner, name, value, on_instance=on_instance))

    def undo(self) -> None:
        while self.rebindings:
            self.rebindings.pop().undo()

    def fallback(self, seam: str, error: Exception | None = None) -> None:
        field = f"{seam}_fallbacks"
        setattr(self.stats, field, getattr(self.stats, field) + 1)
        if error is None:
            return
        self.stats.last_error = f"{type(error).__name__}: {error}"
        if not self.warned:
            self.warned = True
            warnings.warn(f"fused DeepMD dispatch fell back to the stock path: {self.stats.last_error}",
                          RuntimeWarning, stacklevel=4)

    def hit(self, seam: str) -> None:
        field = f"{seam}_hits"
        setattr(self.stats, field, getattr(self.stats, field) + 1)

    # -- softmax ---------------------------------------------------------------
    def softmax(self, stock, logits, edge_env, dst, n_nodes, z_bias_raw, eps, src_weight=None):
        shapes_ok = (src_weight is None and _kernel_operand(logits) and logits.dim() == 3 and logits.shape[0] > 0
                     and _kernel_operand(edge_env) and edge_env.numel() == logits.shape[0]
                     and isinstance(dst, torch.Tensor) and dst.dtype == torch.int64 and dst.dim() == 1
                     and dst.numel() == logits.shape[0] and n_nodes > 0 and isinstance(z_bias_raw, torch.Tensor)
                     and z_bias_raw.numel() == logits.shape[1] * logits.shape[2])
        if not shapes_ok:
            self.fallback("softmax")
            return stock(logits, edge_env, dst, n_nodes, z_bias_raw, eps, src_weight)
        edges, focus, heads = logits.shape
        try:
            offsets, order = self.csr.get(dst, n_nodes)
            null = torch.log(F.softplus(z_bias_raw.reshape(1, focus * heads).to(torch.float32)) + float(eps))
            result = self.ops.segment_softmax(logits.reshape(edges, focus * heads), edge_env.reshape(edges), offsets,
                                              null.expand(n_nodes, focus * heads).contiguous(), order=order)
        except Exception as error:  # noqa: BLE001 -- a seam must never break inference
            self.fallback("softmax", error)
            return stock(logits, edge_env, dst, n_nodes, z_bias_raw, eps, None)
        self.hit("softmax")
        alpha = result[0] if isinstance(result, tuple) else result
        return alpha.reshape(edges, focus, heads)

    # -- envelope --------------------------------------------------------------
    def envelope(self, stock, block, x, edge_cache, radial_feat):
        """``stock`` is the block's own ``forward_envelope``, already bound to it."""
        dst = getattr(edge_cache, "dst", None)
        env = getattr(edge_cache, "edge_env", None)
        inverse = getattr(edge_cache, "inv_sqrt_deg", None)
        gate = getattr(edge_cache, "edge_src_gate", None)
        shapes_ok = (not getattr(block, "training", False) and _kernel_operand(x) and x.dim() == 3
                     and _kernel_operand(env) and _kernel_operand(inverse) and inverse.numel() == x.shape[0]
                     and _index_operand(dst) and dst.numel() > 0 and env.numel() == dst.numel()
                     and (gate is None or _kernel_operand(gate)))
        if not shapes_ok:
            self.fallback("envelope")
            return stock(x, edge_cache, radial_feat)
        try:
            message, _ = block.edge_message(x, edge_cache, radial_feat)
            if not _kernel_operand(message) or message.shape[0] != dst.numel():
                raise ValueError("edge message is not a contiguous fp32 (n_edges, ...) tensor")
            scale = env.reshape(-1) if gate is None else env.reshape(-1) * gate.reshape(-1).to(torch.float32)
            offsets, order = self.csr.get(dst, x.shape[0])
            out = self.ops.segment_sum(message.reshape(dst.numel(), -1), dst, offsets, scale.contiguous(),
                                       inverse.reshape(-1).contiguous(), order=order)
        except Exception as error:  # noqa: BLE001 -- a seam must never break inference
            self.fallback("envelope", error)
            return stock(x, edge_cache, radial_feat)
        self.hit("envelope")
        return out.reshape(x.shape)

    # -- force -----------------------------------------------------------------
    def force(self, stock, g, edge_vec, edge_scatter_index, edge_mask, dst_order, dst_row_ptr, src_order,
              src_row_ptr, n_node_per_frame, optional, n_ext, flag):
        """``(force_flat, atom_virial_flat, frame_virial, None)`` of one frame, or DeepMD's own result.

        Served: one frame (``n_node_per_frame == n_ext``), every edge kept
        (``edge_mask`` absent or all true), an empty optional tensor, float32
        or float64 ``[E, 3]`` values and ``[n_ext + 1]`` CSR pointers.  The
        natural edge order need not be grouped by destination: the values are
        put in ``dst_order`` first.
        """
        args = (g, edge_vec, edge_scatter_index, edge_mask, dst_order, dst_row_ptr, src_order, src_row_ptr,
                n_node_per_frame, optional, n_ext, flag)
        dtypes = (torch.float32, torch.float64)
        try:
            atoms = int(n_ext)
            frame_atoms = int(n_node_per_frame) if not isinstance(n_node_per_frame, torch.Tensor) or \
                n_node_per_frame.numel() == 1 else -1
            shapes_ok = (atoms > 0 and frame_atoms == atoms and _kernel_operand(g, dtypes) and g.dim() == 2
                         and g.shape[1] == 3 and _kernel_operand(edge_vec, (g.dtype,)) and edge_vec.shape == g.shape
                         and all(_index_operand(t) and t.numel() == g.shape[0] for t in (dst_order, src_order))
                         and all(_index_operand(t) and t.numel() == atoms + 1 for t in (dst_row_ptr, src_row_ptr))
                         and (optional is None or (isinstance(optional, torch.Tensor) and optional.numel() == 0)))
            if shapes_ok and edge_mask is not None:
                shapes_ok = bool(torch.as_tensor(edge_mask).all())
        except (TypeError, ValueError, RuntimeError):
            shapes_ok = False
        if not shapes_ok:
            self.fallback("force")
            return stock(*args)
        try:
            # the source slots named by their destination slots (kept per grouping pair, so the
            # operator's blob plan, cached per that tensor, is built once per neighbour graph)
            slot_order, identity = self.force_views.get(dst_order, src_order)
            if identity:
                grouped_g, grouped_v = g, edge_vec.detach()
            else:
                grouped_g = g.index_select(0, dst_order)
                grouped_v = edge_vec.detach().index_select(0, dst_order)
            force, virial = self.ops.force_assembly(grouped_g, grouped_v, None, None, dst_row_ptr, src_row_ptr,
                                                    slot_order)
        except Exception as error:  # noqa: BLE001 -- a seam must never break inference
            self.fallback("force", error)
            return stock(*args)
        self.hit("force")
        return force.reshape(-1), virial.reshape(-1), virial.sum(0, keepdim=True), None


_ACTIVE: _Installation | None = None


def _dispatcher(seam: str, stock: Callable) -> Callable:
    """A function that routes calls to the active installation's ``seam``, or to ``stock`` after uninstall."""
    def dispatch(*args, **kwargs):
        installation = _ACTIVE
        if installation is None:
            return stock(*args, **kwargs)
        return getattr(installation, seam)(stock, *args, **kwargs)

    dispatch.__name__ = dispatch.__qualname__ = f"fused_{seam}"
    return dispatch


def _envelope_method(block: Any, stock: Callable) -> MethodType:
    """``forward_envelope`` for ``block``: the active installation's envelope seam, or ``stock`` (already bound)."""
    def fused_envelope(self, x, edge_cache, radial_feat):
        installation = _ACTIVE
        if installation is None:
            return stock(x, edge_cache, radial_feat)
        return installation.envelope(stock, self, x, edge_cache, radial_feat)

    return MethodType(fused_envelope, block)


def deepmd_patch(module: Any, *, ops: Any = None, softmax: bool = True, envelope: bool = True, force: bool = False,
                 blocks: Iterable[Any] | None = None, namespaces: Iterable[Any] | None = None,
                 force_namespaces: Iterable[tuple[Any, str]] | None = None, verbose: bool = True) -> FusedStats:
    """Bind the operators into ``module`` (a DeepPot, DeepEval or ``nn.Module``); returns its counters.

    ``ops`` bundles ``segment_softmax``, ``segment_sum`` and ``force_assembly``
    (default: this build's ``kernels.segment``; without a usable gfx950
    device nothing is replaced).  ``blocks``, ``namespaces`` (modules holding
    the softmax name) and ``force_namespaces`` (``(module, name)`` pairs)
    override where the seams are looked up -- host tests use them instead of
    importing DeepMD.  An earlier installation is removed first.
    """
    global _ACTIVE

    def say(text: str) -> None:
        if verbose:
            print(f"[deepmd_patch] {text}", flush=True)

    if verbose:
        for line in describe_module(module):
            say(line)
    uninstall()
    root, path = _module_root(module)
    targets = list(blocks) if blocks is not None else _so2_blocks(root)
    stats = FusedStats(blocks=len(targets))
    if path not in ("", "model"):
        say(f"resolved module tree: {path} ({type(root).__name__})")
    ops = _segment_operators() if ops is None else ops
    say(f"operators: {'unavailable' if ops is None else 'kernels.segment'}; "
        f"softmax={softmax} envelope={envelope} force={force}")
    if ops is None:
        say("no usable gfx950 operator library on this host -> nothing replaced")
        return stats
    installation = _Installation(ops, stats)
    _ACTIVE = installation

    if softmax:
        homes = [home for home in (namespaces if namespaces is not None else _importable(_SOFTMAX_HOMES))
                 if hasattr(home, _SOFTMAX_NAME)]
        if not homes:
            uninstall()
            raise ValueError(f"deepmd_patch found no module holding {_SOFTMAX_NAME}")
        routed = _dispatcher("softmax", getattr(homes[0], _SOFTMAX_NAME))
        for home in homes:
            installation.rebind(home, _SOFTMAX_NAME, routed)
            say(f"replace {home.__name__}.{_SOFTMAX_NAME} -> fused_deepmd.fused_softmax")
        stats.bound_softmax = True

    if envelope:
        for block in targets:
            installation.rebind(block, _ENVELOPE_NAME, _envelope_method(block, getattr(block, _ENVELOPE_NAME)),
                                on_instance=True)
        stats.bound_envelope = bool(targets)
        say(f"replace SO2Convolution.forward_envelope on {len(targets)} block(s) -> fused_deepmd.fused_envelope")

    if force:
        pairs = list(force_namespaces) if force_namespaces is not None else [
            (home, name) for module_name, name in _FORCE_HOMES for home in _importable((module_name,))]
        for home, name in pairs:
            if hasattr(home, name):
                installation.rebind(home, name, _dispatcher("force", getattr(home, name)))
                say(f"replace {home.__name__}.{name} -> fused_deepmd.fused_force")
                stats.bound_force = True
        if not stats.bound_force:
            say("force seam: DeepMD's edge_force_virial is not importable here -> not bound")
    say(f"installed: softmax={stats.bound_softmax} envelope={stats.bound_envelope} force={stats.bound_force} "
        f"blocks={stats.blocks}")
    return stats


def uninstall(module: Any = None) -> None:
    """Undo the active installation's rebindings (newest first); harmless when none is active."""
    global _ACTIVE
    installation, _ACTIVE = _ACTIVE, None
    if installation is not None:
        installation.undo()


def installed() -> list[str]:
    """``owner.name`` of every rebinding of the active installation, in the order made."""
    return [] if _ACTIVE is None else [rebinding.label() for rebinding in _ACTIVE.rebindings]


def status(stats: FusedStats | None) -> dict[str, Any]:
    """The counters of an installation as a dict (empty for None)."""
    return {} if stats is None else stats.as_dict()


__all__ = ["FusedStats", "deepmd_patch", "describe_module", "installed", "status", "uninstall"]
