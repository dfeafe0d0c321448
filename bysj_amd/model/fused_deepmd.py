"""Binds the gfx950 segment operators into a loaded DeepMD DPA4/SeZM model.

Restates the seam layer of the reference (python/model/fused_deepmd.py:103-462
of lipengfei1409/bysj) over this build's operators.  DeepMD is not edited; two
of its own dispatch points are rebound and every call keeps a fallback to the
stock implementation:

S1  ``segment_envelope_gated_softmax(logits, edge_env, dst, n_nodes,
    z_bias_raw, eps, src_weight=None)`` -- the eager softmax that
    ``SO2Convolution.attention_weights`` calls.  Served by
    ``kernels.segment_softmax`` with ``null_logit = log(softplus(z_bias) + eps)``
    and the envelope folded into the logit inside the kernel.

S2  ``SO2Convolution.forward_envelope(self, x, edge_cache, radial_feat)`` --
    the attention-free aggregation ``zeros -> index_add_(dst) -> mul_``.
    Served by one ``kernels.segment_sum`` call with ``edge_scale = edge_env *
    edge_src_gate`` and ``node_scale = inv_sqrt_deg``.  Unlike the reference,
    the gradient reaches ``edge_scale`` (DeepMD's envelope depends on the
    coordinates, so forces need it).

Both seams need the destination CSR view of ``dst``.  It is built once per
neighbour graph on the device (``kernels.group_by_source``: a check pass,
a stable radix sort when the list is unsorted, a boundary pass) and cached per ``dst`` tensor object; an entry is
dropped when the tensor is freed or written in place (its version counter
moves), so a recycled storage address can never return a stale view.

Counters of hits and fallbacks are kept in :class:`FusedStats`.  A seam falls
back when its inputs are not what the kernels take (``src_weight`` given,
non-fp32, not on the GPU, non-contiguous, wrong shapes, training mode) or when
the operator raises; the first error is reported once as a warning.
"""
from __future__ import annotations

import warnings
import weakref
from dataclasses import asdict, dataclass, field
from types import MethodType
from typing import Any, Iterable

import torch
import torch.nn.functional as F

_CSR_CAPACITY = 4
# Host tests drive the seams with CPU tensors and a stand-in operator bundle.
# In a real install the device check below keeps CPU tensors on DeepMD's own
# path; only a test lifts it.
_ACCEPT_ANY_DEVICE = False
_SOFTMAX_NAME = "segment_envelope_gated_softmax"


@dataclass
class FusedStats:
    """Hit, fallback and error counters of the installed seams."""

    softmax_hits: int = 0
    softmax_fallbacks: int = 0
    envelope_hits: int = 0
    envelope_fallbacks: int = 0
    bound_softmax: bool = False
    bound_envelope: bool = False
    blocks: int = 0
    last_error: str | None = None

    def as_dict(self) -> dict[str, Any]:
        return asdict(self)


def _fp32_operand(value: Any, dtype: torch.dtype = torch.float32) -> bool:
    """A tensor the kernels accept: right dtype, contiguous, on the GPU."""
    return (isinstance(value, torch.Tensor) and value.dtype == dtype and value.is_contiguous()
            and (value.is_cuda or _ACCEPT_ANY_DEVICE))


def _segment_operators():
    """The operator module of this build (``kernels.segment``) or None if it cannot run."""
    try:
        from ..kernels import segment
    except ImportError:
        try:
            from kernels import segment  # imported as the top-level package `model`
        except ImportError:
            return None
    return segment if segment.segment_available() else None


def _group_by_destination(dst: torch.Tensor, n_nodes: int):
    """``(offsets, order)``, with ``order`` None when ``dst`` is already sorted (natural-order kernels)."""
    try:
        from ..kernels.segment import destination_grouping
    except ImportError:
        from kernels.segment import destination_grouping
    return destination_grouping(dst, n_nodes)


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
            return _group_by_destination(dst, int(n_nodes))
        key = id(dst)
        entry = self._entries.pop(key, None)
        if entry is not None and entry[0]() is dst and entry[1] == stamp:
            self._entries[key] = entry            # most recently used last
            return entry[2], entry[3]
        offsets, order = _group_by_destination(dst, int(n_nodes))
        reference = weakref.ref(dst, lambda _, key=key: self._entries.pop(key, None))
        self._entries[key] = (reference, stamp, offsets, order)
        while len(self._entries) > self.capacity:
            self._entries.pop(next(iter(self._entries)))
        return offsets, order

    def __len__(self) -> int:
        return len(self._entries)


@dataclass
class _Session:
    """One installation: the operators, its counters and the stock softmax."""

    ops: Any
    stats: FusedStats
    reference_softmax: Any
    csr: _CsrView = field(default_factory=_CsrView)
    warned: bool = False

    def _fall_back(self, error: Exception | None = None) -> None:
        if error is not None:
            self.stats.last_error = f"{type(error).__name__}: {error}"
            if not self.warned:
                self.warned = True
                warnings.warn("fused DeepMD dispatch fell back to the stock path: " + self.stats.last_error,
                              RuntimeWarning, stacklevel=4)

    # -- S1 ------------------------------------------------------------------
    def softmax(self, logits, edge_env, dst, n_nodes, z_bias_raw, eps, src_weight=None):
        stock = self.reference_softmax
        if src_weight is not None or not self._softmax_inputs_ok(logits, edge_env, dst, n_nodes, z_bias_raw):
            self.stats.softmax_fallbacks += 1
            self._fall_back()
            return stock(logits, edge_env, dst, n_nodes, z_bias_raw, eps, src_weight)
        n_edges, n_focus, n_head = logits.shape
        channels = n_focus * n_head
        try:
            offsets, order = self.csr.get(dst, n_nodes)
            bias = z_bias_raw.reshape(-1).to(torch.float32)
            null_logit = torch.log(F.softplus(bias) + float(eps)).reshape(1, channels).expand(n_nodes, channels)
            result = self.ops.segment_softmax(logits.reshape(n_edges, channels), edge_env.reshape(n_edges), offsets,
                                              null_logit.contiguous(), order=order)
            alpha = result[0] if isinstance(result, tuple) else result
        except Exception as error:  # noqa: BLE001 -- a seam must never break inference
            self.stats.softmax_fallbacks += 1
            self._fall_back(error)
            return stock(logits, edge_env, dst, n_nodes, z_bias_raw, eps, None)
        self.stats.softmax_hits += 1
        return alpha.reshape(n_edges, n_focus, n_head)

    @staticmethod
    def _softmax_inputs_ok(logits, edge_env, dst, n_nodes, z_bias_raw) -> bool:
        if not (_fp32_operand(logits) and logits.ndim == 3 and logits.shape[0] > 0 and _fp32_operand(edge_env)):
            return False
        if not (isinstance(dst, torch.Tensor) and dst.dtype == torch.int64 and dst.ndim == 1) or n_nodes <= 0:
            return False
        n_edges, n_focus, n_head = logits.shape
        return (isinstance(z_bias_raw, torch.Tensor) and z_bias_raw.numel() == n_focus * n_head
                and edge_env.numel() == n_edges and dst.numel() == n_edges)

    # -- S2 ------------------------------------------------------------------
    def envelope(self, original, block, x, edge_cache, radial_feat):
        """``original`` is the block's stock ``forward_envelope``, already bound."""
        dst = getattr(edge_cache, "dst", None)
        edge_env = getattr(edge_cache, "edge_env", None)
        inverse = getattr(edge_cache, "inv_sqrt_deg", None)
        gate = getattr(edge_cache, "edge_src_gate", None)
        if not self._envelope_inputs_ok(block, x, dst, edge_env, inverse, gate):
            self.stats.envelope_fallbacks += 1
            self._fall_back()
            return original(x, edge_cache, radial_feat)
        n_edges = dst.shape[0]
        try:
            message, _ = block.edge_message(x, edge_cache, radial_feat)
            if not _fp32_operand(message) or message.shape[0] != n_edges:
                raise ValueError("edge message is not a contiguous fp32 (n_edges, ...) tensor")
            weight = edge_env.reshape(-1)
            if gate is not None:
                weight = weight * gate.reshape(-1).to(torch.float32)
            offsets, order = self.csr.get(dst, x.shape[0])
            out = self.ops.segment_sum(message.reshape(n_edges, -1), dst, offsets, weight.contiguous(),
                                       inverse.reshape(-1).contiguous(), order=order)
        except Exception as error:  # noqa: BLE001 -- a seam must never break inference
            self.stats.envelope_fallbacks += 1
            self._fall_back(error)
            return original(x, edge_cache, radial_feat)
        self.stats.envelope_hits += 1
        return out.reshape(x.shape)

    @staticmethod
    def _envelope_inputs_ok(block, x, dst, edge_env, inverse, gate) -> bool:
        if getattr(block, "training", False):
            return False
        if not (_fp32_operand(x) and x.ndim == 3 and _fp32_operand(edge_env) and _fp32_operand(inverse)):
            return False
        if not (_fp32_operand(dst, torch.int64) and dst.ndim == 1 and dst.numel() > 0):
            return False
        if gate is not None and not _fp32_operand(gate):
            return False
        return inverse.numel() == x.shape[0] and edge_env.numel() == dst.numel()


_SESSION: _Session | None = None
# What the installation replaced: "<module>.<name>" -> (module, original) for
# rebound names, "block:<id>" -> (block, instance attribute or None) for
# patched methods (None: the block used its class's method).
_SAVED: dict[str, tuple[Any, Any]] = {}


def _softmax_namespaces() -> list[Any]:
    """DeepMD modules that hold the S1 name (imported only when patching a real model)."""
    import deepmd.pt.model.descriptor.sezm_nn.attention as attention
    import deepmd.pt.model.descriptor.sezm_nn.so2 as so2

    found = [attention, so2]
    try:
        import deepmd.pt.model.descriptor.sezm_nn as package
    except ImportError:  # pragma: no cover
        return found
    return found + [package]


def _blocks(root: Any) -> list[Any]:
    """SO(2) convolution blocks: modules exposing both aggregation seams."""
    return [m for m in root.modules()
            if callable(getattr(m, "edge_message", None)) and callable(getattr(m, "forward_envelope", None))
            and hasattr(m, "_segment_softmax_fn")]


def _module_root(model: Any) -> tuple[Any | None, str]:
    """The ``nn.Module`` tree behind a DeepPot/DeepEval wrapper, and where it was found.

    A module is its own root.  DeepMD's legacy ``pt`` backend keeps the tree at
    ``deep_eval.dp``, the ``pt_expt`` backend at ``deep_eval._dpmodel``.
    """
    if callable(getattr(model, "modules", None)):
        return model, "model"
    deep_eval = getattr(model, "deep_eval", None)
    if deep_eval is None:
        return None, ""
    for name in ("_dpmodel", "dp", "model"):
        candidate = getattr(deep_eval, name, None)
        if candidate is not None and callable(getattr(candidate, "modules", None)):
            return candidate, f"deep_eval.{name}"
    if callable(getattr(deep_eval, "modules", None)):
        return deep_eval, "deep_eval"
    return None, ""


def describe_module(module: Any, *, max_depth: int = 2, max_rows: int = 40) -> list[str]:
    """Printable lines: the module tree (to ``max_depth``) and every patch target."""
    root, path = _module_root(module)
    if root is None:
        return [f"module: {type(module).__name__} (no nn.Module tree found -- expected a module, "
                "or a DeepPot/DeepEval wrapper with deep_eval.dp / deep_eval._dpmodel)",
                "patch targets: 0 (nothing can be bound)"]
    named = list(root.named_modules()) if hasattr(root, "named_modules") else []
    via = "" if path == "model" else f" -> {path}"
    lines = [f"module: {type(module).__name__}{via} ({type(root).__name__}, {len(named)} submodules)"]
    for name, child in named[:max_rows]:
        depth = name.count(".") + 1 if name else 0
        if depth <= max_depth:
            lines.append(f"  {'  ' * depth}{name or '<root>'}  {type(child).__name__}")
    if len(named) > max_rows:
        lines.append(f"  ... {len(named) - max_rows} more submodules")
    targets = _blocks(root)
    lines.append(f"patch targets: {len(targets)} SO(2) block(s)")
    for index, block in enumerate(targets):
        lines.append(f"  [{index}] {type(block).__name__}  n_atten_head={getattr(block, 'n_atten_head', '?')}  "
                     "seams: forward_envelope -> segment_sum, attention softmax -> segment_softmax")
    return lines


def _say(verbose: bool, text: str) -> None:
    if verbose:
        print(f"[deepmd_patch] {text}", flush=True)


def deepmd_patch(module: Any, *, ops: Any = None, softmax: bool = True, envelope: bool = True,
                 blocks: Iterable[Any] | None = None, namespaces: Iterable[Any] | None = None,
                 verbose: bool = True) -> FusedStats:
    """Bind the operators into ``module`` (a DeepPot, DeepEval or ``nn.Module``).

    ``ops`` is a bundle with ``segment_sum`` and ``segment_softmax`` (default:
    this build's ``kernels.segment``; without a usable gfx950 device the call
    replaces nothing).  ``blocks`` and ``namespaces`` override where the seams
    are found (host tests use them instead of importing DeepMD).  Any earlier
    installation is removed first.  Returns the counters of this installation.
    """
    global _SESSION
    stats = FusedStats()
    for line in describe_module(module) if verbose else ():
        _say(True, line)
    uninstall(module)
    root, path = _module_root(module)
    targets = list(blocks) if blocks is not None else (list(_blocks(root)) if root is not None else [])
    if root is not None and path != "model":
        _say(verbose, f"resolved module tree: {path} ({type(root).__name__})")
    stats.blocks = len(targets)
    ops = _segment_operators() if ops is None else ops
    _say(verbose, f"operators: {'kernels.segment' if ops is not None else 'unavailable'}; "
                  f"softmax={softmax} envelope={envelope}")
    if ops is None:
        _say(verbose, "no usable gfx950 operator library on this host -> nothing replaced")
        return stats

    spaces: list[Any] = []
    stock_softmax = None
    if softmax:
        spaces = list(namespaces) if namespaces is not None else _softmax_namespaces()
        if not spaces:
            raise ValueError("deepmd_patch needs at least one namespace holding the softmax seam")
        stock_softmax = getattr(spaces[0], _SOFTMAX_NAME)
    session = _Session(ops=ops, stats=stats, reference_softmax=stock_softmax)
    _SESSION = session

    if softmax:
        def bound_softmax(logits, edge_env, dst, n_nodes, z_bias_raw, eps, src_weight=None):
            active = _SESSION
            if active is None:  # uninstalled while a reference to this function survived
                return stock_softmax(logits, edge_env, dst, n_nodes, z_bias_raw, eps, src_weight)
            return active.softmax(logits, edge_env, dst, n_nodes, z_bias_raw, eps, src_weight)

        for space in spaces:
            if hasattr(space, _SOFTMAX_NAME):
                _SAVED[f"{space.__name__}.{_SOFTMAX_NAME}"] = (space, getattr(space, _SOFTMAX_NAME))
                setattr(space, _SOFTMAX_NAME, bound_softmax)
                _say(verbose, f"replace {space.__name__}.{_SOFTMAX_NAME} -> fused_deepmd.bound_softmax")
        stats.bound_softmax = True

    if envelope:
        for block in targets:
            stock = block.forward_envelope  # bound: called as stock(x, edge_cache, radial_feat)
            _SAVED[f"block:{id(block)}"] = (block, getattr(block, "__dict__", {}).get("forward_envelope"))

            def patched(self, x, edge_cache, radial_feat, _stock=stock):
                active = _SESSION
                if active is None:
                    return _stock(x, edge_cache, radial_feat)
                return active.envelope(_stock, self, x, edge_cache, radial_feat)

            block.forward_envelope = MethodType(patched, block)
        stats.bound_envelope = bool(targets)
        _say(verbose, f"replace SO2Convolution.forward_envelope on {len(targets)} block(s) -> fused_deepmd.patched")
    _say(verbose, f"installed: softmax={stats.bound_softmax} envelope={stats.bound_envelope} blocks={stats.blocks}")
    return stats


def uninstall(module: Any = None) -> None:
    """Restore every rebound name and method; harmless when nothing is installed."""
    global _SESSION
    for key, (owner, original) in list(_SAVED.items()):
        if key.startswith("block:"):
            # the patch is an instance attribute: put back what was there, or
            # delete it so that the class method shows through again
            if original is None:
                owner.__dict__.pop("forward_envelope", None)
            else:
                owner.__dict__["forward_envelope"] = original
        else:
            setattr(owner, key.rsplit(".", 1)[1], original)
    _SAVED.clear()
    _SESSION = None


def status(stats: FusedStats | None) -> dict[str, Any]:
    """The counters of an installation as a dict (empty for None)."""
    return {} if stats is None else stats.as_dict()


__all__ = ["FusedStats", "deepmd_patch", "describe_module", "status", "uninstall"]
