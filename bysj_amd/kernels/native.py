"""Device gate and native-module loader (python/kernels/native.py:9-62 of the reference).

The reference admits Hygon DCU architectures; this build admits the MI355X
(``gfx950``) only.  The gate keeps the reference's name, ``require_dcu``, so
code and tests that patch ``kernels.<op>.require_dcu`` keep working.
"""
from __future__ import annotations

import importlib
import sys

import torch

SUPPORTED_ARCHITECTURES = frozenset({"gfx950"})
_NATIVE_MODULE = __name__.rsplit(".", 1)[0] + "._C"

# Every operator call passes through the gate and the loader, so both keep
# what they have established: the loaded native module (only the one that is
# in sys.modules, i.e. the real import) and the device indices whose
# architecture has been checked.  `importlib.import_module` takes the import
# system's module lock even for a loaded module, which costs tens of
# microseconds per call.
_LOADED = None
_CHECKED_DEVICES: set[int] = set()
_RUNTIME_READY = False


def _require_hip_runtime() -> None:
    # A HIP runtime with a visible device stays so for the process; only the
    # first successful check is paid (torch.cuda.is_available reads the
    # environment on every call).
    global _RUNTIME_READY
    if _RUNTIME_READY:
        return
    if not torch.version.hip:
        raise RuntimeError("gfx950 operators require a ROCm (HIP) build of PyTorch")
    if not torch.cuda.is_available():
        raise RuntimeError("gfx950 operators require a visible MI355X (gfx950) device")
    _RUNTIME_READY = True


def require_dcu(*tensors) -> torch.device:
    """Check the HIP runtime, that every tensor lives on one gfx950 device, and return it.

    ``None`` and non-tensor arguments are skipped.  Raises ``RuntimeError``.
    """
    _require_hip_runtime()
    device = None
    for tensor in tensors:
        if not isinstance(tensor, torch.Tensor):
            continue
        if tensor.device.type != "cuda":
            raise RuntimeError(f"gfx950 operator inputs must be on the GPU, got {tensor.device}")
        if device is not None and tensor.device != device:
            raise RuntimeError("gfx950 operator inputs must share one device")
        device = tensor.device
    index = torch.cuda.current_device() if device is None or device.index is None else device.index
    if index not in _CHECKED_DEVICES:
        try:
            properties = torch.cuda.get_device_properties(index)
        except (AssertionError, RuntimeError) as error:
            raise RuntimeError(f"cannot inspect GPU device {index}") from error
        architecture = str(getattr(properties, "gcnArchName", "")).split(":", 1)[0]
        if architecture not in SUPPORTED_ARCHITECTURES:
            raise RuntimeError(
                f"unsupported GPU architecture {architecture!r}; these operators are built for gfx950 (MI355X)"
            )
        _CHECKED_DEVICES.add(index)
    return torch.device("cuda", index)


def _extension(required_symbol: str):
    """Import the native module and require one of its entry points."""
    global _LOADED
    _require_hip_runtime()
    extension = _LOADED
    if extension is None:
        try:
            extension = importlib.import_module(_NATIVE_MODULE)
        except (ImportError, OSError) as error:
            raise RuntimeError(
                "the gfx950 operator library is not built: run __graft_entry__.build() "
                "(segment, GIE and RMSNorm operators)"
            ) from error
        if sys.modules.get(_NATIVE_MODULE) is extension:
            _LOADED = extension
    if not hasattr(extension, required_symbol):
        raise RuntimeError(f"the loaded {_NATIVE_MODULE} has no {required_symbol!r} entry point")
    return extension


class _Untracked:
    """Stands in for an autograd context when no gradient can flow.

    The operators' ``Function.forward`` methods run unchanged on it: what they
    would save for the backward is dropped, and ``needs_input_grad`` is all
    False (so a forward that writes extra state only for its backward skips
    it).
    """

    def __init__(self, count: int):
        self.needs_input_grad = (False,) * count

    def save_for_backward(self, *tensors) -> None:
        pass


def version_stamp(tensor: torch.Tensor):
    """``(storage address, version counter, numel, device)`` of ``tensor``, or None for an inference tensor.

    The caches of derived data (degree plans, groupings) use the stamp to see
    in-place writes.  Tensors made under ``torch.inference_mode`` keep no
    version counter, so their in-place writes cannot be seen: callers derive
    afresh from them instead of caching.
    """
    if tensor.is_inference():
        return None
    return (tensor.data_ptr(), tensor._version, tensor.numel(), tensor.device)


def apply_function(function, *args):
    """``function.apply(*args)``, or its forward alone when no argument needs a gradient.

    Outside grad mode (``torch.no_grad``, ``torch.inference_mode``) or when
    no tensor argument requires a gradient, ``apply`` would record nothing:
    calling the forward directly gives the same tensors without the autograd
    bookkeeping, which is most of the Python layer's cost per eager call.
    """
    if torch.is_grad_enabled() and any(isinstance(a, torch.Tensor) and a.requires_grad for a in args):
        return function.apply(*args)
    return function.forward(_Untracked(len(args)), *args)
