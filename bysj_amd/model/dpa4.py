"""``DPA4Model``: DeepMD's ``DeepPot`` with the fused seams (python/model/dpa4.py:81-190 of the reference).

DeepMD-kit owns the DPA4/SeZM graph, checkpoint loading, neighbour lists and
the energy/force/virial evaluation; this wrapper adds the ``fused=`` switch,
which installs seams of :mod:`fused_deepmd`, and a lifecycle that removes
them again before the ``DeepPot`` is closed.

Seams: ``softmax`` and ``envelope`` (the reference's two) and ``force`` (this
build's third, DeepMD's edge force/virial assembly).  ``fused=True`` selects
the reference's two; ``force`` is selected by name.
"""
from __future__ import annotations

import os
from collections.abc import Iterable, Mapping
from pathlib import Path
from typing import Any

# seam -> selected by fused=True
_SEAM_TABLE = {"softmax": True, "envelope": True, "force": False}
SEAMS = tuple(_SEAM_TABLE)

# Keywords of earlier releases: a call site still passing one must fail before
# anything is loaded, not have the keyword forwarded to DeepPot.
_RETIRED_KEYWORDS = {
    "tilelang_ops": "drop the argument; TileLang dispatch is not part of this operator slice",
    "native_ops": "drop the argument and select seams with fused=(\"softmax\", \"envelope\")",
}

# DeepPot methods the wrapper passes through unchanged
_PASS_THROUGH = ("get_rcut", "get_type_map", "get_ntypes", "get_model_def_script")


def _seam_name(name: Any) -> str:
    key = name.strip().lower() if isinstance(name, str) else None
    if key not in _SEAM_TABLE:
        raise ValueError(f"unknown fused seam {name!r}; choose from: {', '.join(SEAMS)}")
    return key


def _normalize_fused(fused: Any) -> dict[str, bool] | None:
    """The per-seam switches of a ``fused`` argument, or None to install nothing.

    Any false value (``None``, ``False``, ``0``, ``""``, an empty collection)
    installs nothing.  ``True`` selects the default seams; a name, or a
    collection of names, selects those (the result names only them); a
    mapping gives every default seam a switch, off unless the mapping turns
    it on, plus any other seam it names.  Unknown names raise
    ``ValueError``, other argument types ``TypeError``.
    :func:`_patch_switches` turns a selection into the switch of every seam.
    """
    if not fused:
        return None
    if fused is True:
        return {name: True for name, default in _SEAM_TABLE.items() if default}
    if isinstance(fused, Mapping):
        named = {_seam_name(name): bool(value) for name, value in fused.items()}
        selection = {name: named.pop(name, False) for name, default in _SEAM_TABLE.items() if default}
        selection.update(named)
        return selection
    if isinstance(fused, str):
        return {_seam_name(fused): True}
    if isinstance(fused, Iterable):
        return {_seam_name(name): True for name in fused} or None
    raise TypeError("fused must be a bool, a seam name, a collection of seam names or a mapping")


def _patch_switches(selection: Mapping[str, bool]) -> dict[str, bool]:
    """``deepmd_patch``'s keyword for every seam: on only where ``selection`` turns it on.

    ``deepmd_patch`` switches the reference's two seams on by default, so a
    selection of one seam must switch the others off explicitly.
    """
    return {name: bool(selection.get(name, False)) for name in SEAMS}


def _create_deep_pot(model_file: str, **kwargs: Any) -> Any:
    """``deepmd.infer.DeepPot(model_file, **kwargs)``, imported only when a model is opened."""
    try:
        from deepmd.infer import DeepPot
    except ImportError as error:
        raise RuntimeError("DPA4Model needs DeepMD-kit with its PyTorch inference backend installed") from error
    return DeepPot(model_file, **kwargs)


def _backend_name(deep_pot: Any) -> str:
    """The DeepMD backend running ``deep_pot`` (``pt``, ``pt_expt``, ...): the package under ``deepmd``."""
    module = type(getattr(deep_pot, "deep_eval", None)).__module__
    top, _, rest = module.partition(".")
    return rest.partition(".")[0] if top == "deepmd" and rest else "unknown"


def _seam_module():
    try:
        from . import fused_deepmd
    except ImportError:  # pragma: no cover -- imported as a top-level package
        import fused_deepmd
    return fused_deepmd


class DPA4Model:
    """DeepMD ``DeepPot`` that can bind the gfx950 segment operators.

    ``fused``: ``True``, a seam name, a collection of names or a mapping
    (see :func:`_normalize_fused`); ``None``/``False`` leaves DeepMD as it
    is.  Remaining keyword arguments go to ``deepmd.infer.DeepPot``.
    ``fused_ops`` holds the installation's counters, ``fused_seams`` the
    selection, ``backend`` DeepMD's backend name.
    """

    def __init__(self, model_file: str | os.PathLike[str], *, fused: Any = None, **deepmd_kwargs: Any) -> None:
        retired = [keyword for keyword in _RETIRED_KEYWORDS if keyword in deepmd_kwargs]
        if retired:
            keyword = retired[0]
            raise RuntimeError(f"{keyword} was removed from DPA4Model: {_RETIRED_KEYWORDS[keyword]}")
        self.model_file = str(Path(model_file).expanduser())
        self.fused_seams = _normalize_fused(fused)  # before the checkpoint is read
        self._deep_pot = _create_deep_pot(self.model_file, **deepmd_kwargs)
        self.backend = _backend_name(self._deep_pot)
        self.fused_ops: dict[str, Any] = {}
        if self.fused_seams:
            seams = _seam_module()
            self.fused_ops = dict(seams.status(seams.deepmd_patch(self._deep_pot,
                                                                  **_patch_switches(self.fused_seams))))

    def eval(self, coords: Any, cells: Any, atom_types: Any, *, atomic: bool = False, fparam: Any = None,
             aparam: Any = None, **kwargs: Any) -> Any:
        """Energies, forces and virials from DeepMD's ``DeepPot.eval`` (every argument forwarded)."""
        return self._deep_pot.eval(coords, cells, atom_types, atomic=atomic, fparam=fparam, aparam=aparam, **kwargs)

    predict = eval
    __call__ = eval

    def close(self) -> None:
        """Remove the installed seams (the first time only), then close the DeepPot."""
        if self.fused_ops:
            self.fused_ops = {}
            _seam_module().uninstall(self._deep_pot)
        close = getattr(self._deep_pot, "close", None)
        if callable(close):
            close()

    def __enter__(self) -> "DPA4Model":
        return self

    def __exit__(self, *exc_info: Any) -> None:
        self.close()

    def __repr__(self) -> str:
        fields = {"model_file": self.model_file, "backend": self.backend, "fused_ops": self.fused_ops}
        return "DPA4Model(" + ", ".join(f"{key}={value!r}" for key, value in fields.items()) + ")"


def _pass_through(name: str):
    def method(self: DPA4Model, *args: Any, **kwargs: Any) -> Any:
        return getattr(self._deep_pot, name)(*args, **kwargs)

    method.__name__ = method.__qualname__ = name
    method.__doc__ = f"``DeepPot.{name}`` of the wrapped model."
    return method


for _name in _PASS_THROUGH:
    setattr(DPA4Model, _name, _pass_through(_name))
del _name

__all__ = ["DPA4Model", "SEAMS"]
