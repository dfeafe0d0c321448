"""ctypes binding of libdpa4k.so (the C ABI declared in include/dpa4k.h).

The library is loaded lazily, after torch, so that its dependency on
``libamdhip64.so.7`` resolves to the HIP runtime torch already loaded: one
runtime per process, torch's streams and allocations valid in both.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

# bysj_amd/libdpa4k.so, one directory above this package (also when the package
# is imported under its reference name, `kernels`, with bysj_amd/ on sys.path).
LIBRARY_PATH = Path(__file__).resolve().parent.parent / "libdpa4k.so"

OK, EINVAL, EHIP, EWORKSPACE = 0, 1, 2, 3
ABI_VERSION = 10

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_SZ = ctypes.c_size_t
_F32 = ctypes.c_float
_INT = ctypes.c_int



class EdgeOperand(ctypes.Structure):
    """``dpa4k_edge_operand``: an fp32 view over (edge, row, channel) with element strides."""

    _fields_ = [("data", ctypes.c_void_p), ("stride", ctypes.c_int64 * 3)]


_OPERANDS = ctypes.POINTER(EdgeOperand)

# name -> (restype, argtypes); mirrors include/dpa4k.h one to one.
PROTOTYPES: dict[str, tuple[object, list[object]]] = {
    "dpa4k_last_error": (ctypes.c_char_p, []),
    "dpa4k_abi_version": (_INT, []),
    "dpa4k_segment_offsets_workspace_size": (_SZ, [_I64, _I64]),
    "dpa4k_segment_offsets": (_INT, [_P, _I64, _I64, _P, _P, _SZ, _P]),
    "dpa4k_group_by_key_workspace_size": (_SZ, [_I64, _I64]),
    "dpa4k_group_by_key": (_INT, [_P, _I64, _I64, _P, _P, _P, _SZ, _P]),
    "dpa4k_segment_offsets_async": (_INT, [_P, _I64, _I64, _P, _P, _P, _SZ, _P]),
    "dpa4k_group_by_key_async": (_INT, [_P, _I64, _I64, _P, _P, _P, _P, _SZ, _P]),
    "dpa4k_segment_sum_forward": (_INT, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P]),
    "dpa4k_segment_sum_backward": (
        _INT, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P]),
    "dpa4k_segment_softmax_forward": (_INT, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P]),
    "dpa4k_segment_softmax_backward": (
        _INT, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P]),
    "dpa4k_segment_softmax_plan_size": (_SZ, [_I64]),
    "dpa4k_segment_softmax_plan": (
        _INT, [_P, _I64, _I64, _I64, _P, _SZ, ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64), _P]),
    "dpa4k_segment_softmax_forward_planned": (
        _INT, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P, _I64, _I64, _P]),
    "dpa4k_segment_softmax_backward_planned": (
        _INT, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P, _I64, _I64, _P]),
    "dpa4k_force_assembly_f32": (_INT, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _P]),
    "dpa4k_force_assembly_f64": (_INT, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _P]),
    "dpa4k_force_assembly_plan_size": (_SZ, [_I64, _I64, _I64]),
    "dpa4k_force_assembly_plan_workspace_size": (_SZ, [_I64, _I64]),
    "dpa4k_force_assembly_records_size": (_SZ, [_I64, _I64, _I64]),
    "dpa4k_force_assembly_plan": (
        _INT, [_P, _P, _P, _P, _I64, _I64, _I64, _P, _SZ, _P, _SZ, ctypes.POINTER(ctypes.c_int64), _P]),
    "dpa4k_force_assembly_f32_planned": (_INT, [_P, _P, _P, _P, _I64, _I64, _P, _SZ, _P, _SZ, _I64, _I64, _P, _P]),
    "dpa4k_force_assembly_f64_planned": (_INT, [_P, _P, _P, _P, _I64, _I64, _P, _SZ, _P, _SZ, _I64, _I64, _P, _P]),
    "dpa4k_gie_group_workspace_size": (_SZ, [_I64, _I64]),
    "dpa4k_gie_group": (
        _INT, [_P, _P, _I64, _I64, _I64, _I64, _P, _P, ctypes.POINTER(ctypes.c_int32), _P, _SZ, _P]),
    "dpa4k_gie_zonal_scatter_forward_csr": (
        _INT, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, ctypes.c_int32, _P]),
    "dpa4k_gie_zonal_scatter_backward_csr": (
        _INT, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, ctypes.c_int32, _P]),
    "dpa4k_gie_zonal_scatter_forward": (
        _INT, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _SZ, _P]),
    "dpa4k_gie_zonal_scatter_backward": (
        _INT, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _SZ, _P]),
    "dpa4k_gie_workspace_size": (_SZ, [_I64, _I64]),
    "dpa4k_gie_rmsnorm_supported": (_INT, [_I64, _I64]),
    "dpa4k_gie_rmsnorm_forward_csr": (
        _INT, [_P, _P, _P, _P, _P, _P, _P, _F32, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P]),
    "dpa4k_rmsnorm_forward": (_INT, [_P, _P, _P, _P, _I64, _I64, _F32, _P]),
    "dpa4k_rmsnorm_backward_workspace_size": (_SZ, [_I64, _I64]),
    "dpa4k_rmsnorm_backward": (_INT, [_P, _P, _P, _P, _P, _P, _I64, _I64, _P, _SZ, _P]),
    "dpa4k_rmsnorm_backward_noalloc": (_INT, [_P, _P, _P, _P, _P, _P, _I64, _I64, _P]),
    "dpa4k_edge_stream_combine": (
        _INT, [_OPERANDS, _OPERANDS, ctypes.POINTER(_F32), _INT, _INT, _OPERANDS, ctypes.POINTER(ctypes.c_int32), _P,
               _I64, _I64, _I64, _P]),
    "dpa4k_stream_calibrate": (_INT, [_P, _I64, _P, _I64, _P]),
    "dpa4k_set_launch_row_limit": (_INT, [_I64]),
}

_LOCK = threading.Lock()
_LIBRARY: ctypes.CDLL | None = None


class NativeError(RuntimeError):
    """A libdpa4k call returned a non-zero status."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


class NativeIndexError(NativeError, ValueError):
    """An index tensor held values outside its range (status EINVAL)."""


def load() -> ctypes.CDLL:
    """Load libdpa4k.so once and declare every prototype; ImportError if absent."""
    global _LIBRARY
    if _LIBRARY is not None:
        return _LIBRARY
    with _LOCK:
        if _LIBRARY is not None:
            return _LIBRARY
        if not LIBRARY_PATH.exists():
            raise ImportError(
                f"{LIBRARY_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'`"
            )
        import torch  # noqa: F401  -- binds libamdhip64.so.7 to torch's runtime first

        library = ctypes.CDLL(str(LIBRARY_PATH))
        for name, (restype, argtypes) in PROTOTYPES.items():
            function = getattr(library, name)
            function.restype = restype
            function.argtypes = argtypes
        version = library.dpa4k_abi_version()
        if version != ABI_VERSION:
            raise ImportError(f"libdpa4k ABI {version} does not match the binding's {ABI_VERSION}")
        _LIBRARY = library
        return library


def exported_symbols() -> list[str]:
    """Every symbol the binding declares (used by the ABI tests)."""
    return list(PROTOTYPES)


def check(status: int, *, index_error: bool = False) -> None:
    """Raise on a non-zero status with the library's thread-local message."""
    if status == OK:
        return
    message = (_LIBRARY.dpa4k_last_error() or b"").decode(errors="replace") if _LIBRARY else ""
    if index_error and status == EINVAL:
        raise NativeIndexError(status, message)
    raise NativeError(status, message or f"libdpa4k status {status}")
