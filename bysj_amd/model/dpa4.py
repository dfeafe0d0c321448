"""``DPA4Model``: a DeepMD ``DeepPot`` facade with the fused seams (python/model/dpa4.py:81-190 of the reference).

DeepMD-kit owns the DPA4/SeZM graph, checkpoint loading, neighbour lists and
the energy/force/virial; the facade adds the ``fused=`` switch, which installs
the seams of :mod:`fused_deepmd`, and a close/context-manager lifecycle that
uninstalls them before the ``DeepPot`` is closed.
"""
from __future__ import annotations

import os
from pathlib import Path
from typing import Any

SEAMS = ("softmax", "envelope")
_REMOVED_KEYWORDS = {
    "tilelang_ops": "drop the argument; TileLang dispatch is not part of this operator slice",
    "native_ops": "drop the argument and use fused=(\"softmax\", \"envelope\") instead",
}


def _normalize_fused(fused: Any) -> dict[str, bool] | None:
    """Per-seam switches of the ``fused`` argument (None: install nothing).

    ``True`` selects every seam; a seam name or a collection of names selects
    those; a mapping gives each seam explicitly.  Unknown names raise
    ``ValueError``, other types ``TypeError``.
    """
    if not fused:
        return None
    if fused is True:
        return dict.fromkeys(SEAMS, True)
    if isinstance(fused, str):
        fused = (fused,)
    if isinstance(fused, dict):
        unknown = sorted(map(str, set(fused) - set(SEAMS)))
        if unknown:
            raise ValueError(f"unknown fused seams: {', '.join(unknown)}; choose from: {', '.join(SEAMS)}")
        return {name: bool(fused.get(name, False)) for name in SEAMS}
    if isinstance(fused, (list, tuple, set, frozenset)):
        chosen = {}
        for name in fused:
            key = name.strip().lower() if isinstance(name, str) else None
            if key not in SEAMS:
                raise ValueError(f"unknown fused seam {name!r}; choose from: {', '.join(SEAMS)}")
            chosen[key] = True
        return chosen
    raise TypeError("fused must be a bool, a seam name, a sequence of names or a mapping")


def _create_deep_pot(model_file: str, **kwargs: Any) -> Any:
    """Load DeepMD lazily: importing the facade must not require DeepMD."""
    try:
        from deepmd.infer import DeepPot
    except ImportError as error:
        raise RuntimeError("DPA4Model requires an installed DeepMD-kit with the PyTorch inference backend") from error
    return DeepPot(model_file, **kwargs)


def _backend_name(deep_pot: Any) -> str:
    """``pt`` / ``pt_expt`` from the module of DeepPot's evaluator, else ``unknown``."""
    parts = type(getattr(deep_pot, "deep_eval", None)).__module__.split(".")
    return parts[1] if len(parts) >= 2 and parts[0] == "deepmd" else "unknown"


def _fused_module():
    try:
        from . import fused_deepmd
    except ImportError:  # pragma: no cover
        import fused_deepmd
    return fused_deepmd


class DPA4Model:
    """``DeepPot`` facade that can bind the gfx950 segment operators.

    ``fused``: ``True`` installs every seam, a name or a sequence of names
    (``"softmax"``, ``"envelope"``) selects seams, a mapping sets each one,
    ``None``/``False`` leaves DeepMD untouched.  Other keyword arguments go to
    ``deepmd.infer.DeepPot``.
    """

    def __init__(self, model_file: str | os.PathLike[str], *, fused: Any = None, **deepmd_kwargs: Any) -> None:
        self.model_file = str(Path(model_file).expanduser())
        for keyword, hint in _REMOVED_KEYWORDS.items():
            if keyword in deepmd_kwargs:
                raise RuntimeError(f"{keyword} was removed from DPA4Model: {hint}; an old call site should fail "
                                   "loudly instead of being forwarded to DeepPot")
        # validate the switch before a possibly large checkpoint is read
        self.fused_seams = _normalize_fused(fused)
        self._deep_pot = _create_deep_pot(self.model_file, **deepmd_kwargs)
        self.backend = _backend_name(self._deep_pot)
        self.fused_ops: dict[str, Any] = {}
        if self.fused_seams:
            fused_deepmd = _fused_module()
            self.fused_ops = dict(fused_deepmd.status(fused_deepmd.deepmd_patch(self._deep_pot, **self.fused_seams)))

    def eval(self, coords: Any, cells: Any, atom_types: Any, *, atomic: bool = False, fparam: Any = None,
             aparam: Any = None, **kwargs: Any) -> Any:
        """Energy, forces and virial through DeepMD's public ``DeepPot.eval``."""
        return self._deep_pot.eval(coords, cells, atom_types, atomic=atomic, fparam=fparam, aparam=aparam, **kwargs)

    predict = eval
    __call__ = eval

    def get_rcut(self) -> float:
        return self._deep_pot.get_rcut()

    def get_type_map(self) -> list[str]:
        return self._deep_pot.get_type_map()

    def get_ntypes(self) -> int:
        return self._deep_pot.get_ntypes()

    def get_model_def_script(self) -> Any:
        return self._deep_pot.get_model_def_script()

    def close(self) -> None:
        """Uninstall the seams (once), then close the DeepPot."""
        if self.fused_ops:
            _fused_module().uninstall(self._deep_pot)
            self.fused_ops = {}
        closer = getattr(self._deep_pot, "close", None)
        if callable(closer):
            closer()

    def __enter__(self) -> "DPA4Model":
        return self

    def __exit__(self, *exc: Any) -> None:
        self.close()

    def __repr__(self) -> str:
        return f"DPA4Model(model_file={self.model_file!r}, backend={self.backend!r}, fused_ops={self.fused_ops!r})"


__all__ = ["DPA4Model"]
