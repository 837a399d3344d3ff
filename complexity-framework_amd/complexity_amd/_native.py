"""ctypes binding of ``libtrmoe.so`` (the C ABI declared in ``include/trmoe.h``).

Loading is lazy and failures are remembered with their reason, so that the
engine can report them (``HIP_LOAD_ERROR``) and so that every product entry
point that needs the library raises instead of silently doing other work.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Optional

LIB_PATH = Path(
    os.environ.get("TRMOE_LIBRARY", str(Path(__file__).resolve().parent / "lib" / "libtrmoe.so"))
)

ABI_VERSION = 1

OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_HIP = 0, 1, 2, 3
F32, BF16, FP8_E4M3 = 0, 1, 2
ORDER_TOKEN, ORDER_ASSIGNMENT = 0, 1
PACK_GATE_UP, PACK_PLAIN = 0, 1

_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_c_vp = ctypes.c_void_p
_c_size = ctypes.c_size_t
_c_float = ctypes.c_float

# name -> (restype, argtypes); mirrors include/trmoe.h exactly
class CallExtras(ctypes.Structure):
    """trmoe_call_extras (include/trmoe.h): optional extras of the *_ex calls."""

    _fields_ = [
        ("row_scale", ctypes.c_void_p),
        ("rms_eps", ctypes.c_float),
        ("w_frag", ctypes.c_void_p),
        ("w_frag_cols", ctypes.c_int64),
    ]


_c_extras = ctypes.POINTER(CallExtras)

SIGNATURES = {
    "trmoe_abi_version": (_c_int, []),
    "trmoe_last_error": (ctypes.c_char_p, []),
    "trmoe_device_supported": (_c_int, []),
    "trmoe_pack_dims": (_c_int, [_c_int, _c_i64, _c_i64, _c_i64, ctypes.POINTER(_c_i64), ctypes.POINTER(_c_i64)]),
    "trmoe_pack_weight": (
        _c_int,
        [_c_int, _c_int, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
         _c_vp, _c_vp, _c_i64, _c_i64, _c_vp, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp],
    ),
    "trmoe_dense_routed_features": (_c_i64, [_c_i64, _c_int, _c_i64]),
    "trmoe_dense_routed_gate_up": (
        _c_int,
        [_c_int, _c_int, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp, _c_i64, _c_int, _c_i64, _c_vp,
         _c_vp, _c_i64, _c_int, _c_vp, _c_float, _c_float, _c_vp, _c_i64, _c_vp],
    ),
    "trmoe_route_sort_workspace_bytes": (_c_size, [_c_i64, _c_int, _c_int, _c_int]),
    "trmoe_route_sort": (
        _c_int,
        [_c_vp, _c_i64, _c_vp, _c_i64, _c_int, _c_int, _c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
         _c_vp, _c_size, _c_vp],
    ),
    "trmoe_stream_read": (_c_int, [_c_vp, _c_i64, _c_vp, _c_int, _c_vp]),
    "trmoe_route_sort_noalloc": (
        _c_int,
        [_c_vp, _c_i64, _c_vp, _c_i64, _c_int, _c_int, _c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp],
    ),
    "trmoe_shared_gate_up": (
        _c_int,
        [_c_int, _c_int, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp],
    ),
    "trmoe_routed_experts_workspace_bytes": (_c_size, [_c_int, _c_i64, _c_i64]),
    "trmoe_routed_experts": (
        _c_int,
        [_c_int, _c_int, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp, _c_int, _c_int, _c_vp, _c_vp,
         _c_vp, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_size, _c_vp],
    ),
    "trmoe_shared_down_combine_workspace_bytes": (_c_size, [_c_int, _c_i64, _c_i64, _c_i64]),
    "trmoe_shared_down_combine": (
        _c_int,
        [_c_int, _c_int, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp,
         _c_int, _c_vp, _c_float, _c_float, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_size, _c_vp],
    ),
    "trmoe_combine": (
        _c_int,
        [_c_int, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp, _c_int, _c_vp, _c_float, _c_vp, _c_i64,
         _c_vp, _c_i64, _c_vp],
    ),
    "trmoe_rms_row_scale": (_c_int, [_c_int, _c_vp, _c_i64, _c_i64, _c_i64, _c_float, _c_vp, _c_vp]),
    "trmoe_rmsnorm_forward": (
        _c_int, [_c_int, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_float, _c_vp, _c_i64, _c_vp, _c_vp]),
    "trmoe_rmsnorm_backward_workspace_bytes": (_c_size, [_c_int, _c_i64, _c_i64]),
    "trmoe_quantize_rows_e4m3": (
        _c_int, [_c_int, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp, _c_vp]),
    "trmoe_shared_gate_up_a8": (
        _c_int, [_c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp]),
    "trmoe_shared_gate_up_a8_mx": (
        _c_int, [_c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp]),
    "trmoe_shared_down_combine_a8": (
        _c_int,
        [_c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_int, _c_vp,
         _c_float, _c_float, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp],
    ),
    "trmoe_rmsnorm_backward": (
        _c_int,
        [_c_int, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64,
         _c_vp, _c_vp, _c_size, _c_vp],
    ),
    "trmoe_shared_gate_up_rms": (
        _c_int,
        [_c_int, _c_int, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp, _c_i64, _c_vp, _c_float, _c_vp, _c_i64,
         _c_vp],
    ),
    "trmoe_dense_routed_gate_up_rms": (
        _c_int,
        [_c_int, _c_int, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp, _c_i64, _c_int, _c_i64, _c_vp,
         _c_vp, _c_i64, _c_int, _c_vp, _c_float, _c_float, _c_vp, _c_float, _c_vp, _c_i64, _c_vp],
    ),
    "trmoe_routed_experts_rms": (
        _c_int,
        [_c_int, _c_int, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp, _c_int, _c_int, _c_vp, _c_vp,
         _c_vp, _c_vp, _c_i64, _c_vp, _c_vp, _c_i64, _c_vp, _c_size, _c_vp],
    ),
    "trmoe_fragment_bytes": (_c_size, [_c_int, _c_i64, _c_i64]),
    "trmoe_pack_fragments": (_c_int, [_c_int, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp]),
    "trmoe_shared_gate_up_ex": (
        _c_int,
        [_c_int, _c_int, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp, _c_i64, _c_vp, _c_i64, _c_extras, _c_vp],
    ),
    "trmoe_dense_routed_gate_up_ex": (
        _c_int,
        [_c_int, _c_int, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp, _c_i64, _c_int, _c_i64, _c_vp,
         _c_vp, _c_i64, _c_int, _c_vp, _c_float, _c_float, _c_vp, _c_i64, _c_extras, _c_vp],
    ),
    "trmoe_shared_down_combine_ex": (
        _c_int,
        [_c_int, _c_int, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp,
         _c_int, _c_vp, _c_float, _c_float, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_size, _c_extras, _c_vp],
    ),
    "trmoe_shared_gate_up_save": (
        _c_int,
        [_c_int, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp],
    ),
    "trmoe_dense_routed_gate_up_save": (
        _c_int,
        [_c_int, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _c_int, _c_i64, _c_vp, _c_vp, _c_i64, _c_int,
         _c_vp, _c_float, _c_float, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp],
    ),
    "trmoe_shared_swiglu_backward": (
        _c_int,
        [_c_int, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp, _c_i64, _c_float, _c_vp,
         _c_i64, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp],
    ),
    "trmoe_dense_routed_swiglu_backward": (
        _c_int,
        [_c_int, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp, _c_i64, _c_int, _c_i64,
         _c_vp, _c_vp, _c_i64, _c_int, _c_vp, _c_float, _c_float, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp,
         _c_i64, _c_vp],
    ),
    "trmoe_routed_swiglu_backward": (
        _c_int,
        [_c_int, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp, _c_int, _c_int, _c_vp,
         _c_vp, _c_i64, _c_vp, _c_float, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp],
    ),
    "trmoe_weight_grad_workspace_bytes": (_c_size, [_c_int, _c_i64, _c_i64, _c_int, _c_i64]),
    "trmoe_weight_grad": (
        _c_int,
        [_c_int, _c_vp, _c_i64, _c_i64, _c_vp, _c_i64, _c_i64, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64,
         _c_i64, _c_vp, _c_int, _c_vp, _c_i64, _c_i64, _c_vp, _c_size, _c_vp],
    ),
    "trmoe_weight_grad_mapped_workspace_bytes": (_c_size, [_c_int, _c_i64, _c_i64, _c_i64]),
    "trmoe_weight_grad_mapped": (
        _c_int,
        [_c_int, _c_vp, _c_i64, _c_i64, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_vp, _c_vp,
         _c_vp, _c_i64, _c_vp, _c_size, _c_vp],
    ),
    "trmoe_grouped_linear": (
        _c_int,
        [_c_int, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_int, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp],
    ),
}

_lib: Optional[ctypes.CDLL] = None
_load_error: Optional[str] = None


class TRMoEError(RuntimeError):
    """A libtrmoe call returned a failure status."""

    def __init__(self, status: int, where: str, message: str):
        super().__init__(f"{where}: {message} (status {status})")
        self.status = status


def load(path: Optional[Path] = None) -> ctypes.CDLL:
    """Load and bind the library once; raise RuntimeError with the cause on failure."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    target = Path(path) if path is not None else LIB_PATH
    try:
        lib = ctypes.CDLL(str(target))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.trmoe_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"ABI version {version} != expected {ABI_VERSION}")
    except (OSError, AttributeError, RuntimeError) as exc:
        _load_error = f"cannot load {target}: {exc}"
        raise RuntimeError(_load_error) from exc
    _lib = lib
    _load_error = None
    return lib


def available() -> bool:
    try:
        load()
        return True
    except RuntimeError:
        return False


def load_error() -> Optional[str]:
    if _lib is None and _load_error is None:
        available()
    return _load_error


def check(status: int, where: str) -> None:
    if status != OK:
        msg = _lib.trmoe_last_error().decode("utf-8", "replace") if _lib is not None else "?"
        if status == ERR_INVALID:
            raise ValueError(f"{where}: {msg}")
        if status == ERR_UNSUPPORTED:
            raise NotImplementedError(f"{where}: {msg}")
        raise TRMoEError(status, where, msg)
