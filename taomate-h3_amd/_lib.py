"""ctypes binding of libtaomate_h3_amd.so (the C ABI in include/taomate_h3_amd.h).

There is no fallback: if the library is missing or fails to load, every
operation raises.  Build it with ``python taomate-h3_amd/build.py`` (or
``__graft_entry__.build()``).
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libtaomate_h3_amd.so"

# Entry points and their C signatures (names exactly as in the header).
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float
SIGNATURES: dict[str, tuple[type | None, list]] = {
    "h3q_version": (_I, []),
    "h3q_last_error": (ctypes.c_char_p, []),
    "h3q_quant_rows": (_I, [_P, _I64, _I64, _I64, _I, _I, _P, _I64, _P, _P]),
    "h3q_quant_tensor_workspace_floats": (_I64, [_I64, _I64]),
    "h3q_quant_tensor_e4m3": (_I, [_P, _I64, _I64, _I64, _P, _P, _P, _I64, _P, _P]),
    "h3q_quant_tensor_e4m3_bf16_divisor": (_I, [_P, _I64, _I64, _I64, _P, _P, _P, _I64, _P, _P]),
    "h3q_quant_tensor_e4m3_noalloc": (_I, [_P, _I64, _I64, _I64, _P, _P, _I64, _P, _P]),
    "h3q_quant_tensor_e4m3_typed": (_I, [_P, _I, _I, _I64, _I64, _I64, _P, _P, _P, _I64, _P, _P]),
    "h3q_swiglu_quant": (_I, [_P, _I64, _I64, _I64, _P, _I64, _I, _I, _P, _I64, _P, _P]),
    "h3q_quant_per_head_workspace_floats": (_I64, [_I64, _I64, _I64, _I64]),
    "h3q_quant_per_head_e4m3": (_I, [_P, _I64, _I64, _I64, _I64, _P, _P, _P, _P]),
    "h3q_tiled_bytes": (_I64, [_I64, _I64]),
    "h3q_quant_rows_tiled": (_I, [_P, _I64, _I64, _I64, _I, _I, _I64, _P, _P, _P]),
    "h3q_scaled_mm": (_I, [_I, _P, _I64, _I, _P, _I, _P, _I64, _I, _P, _I, _P, _P, _I64, _P, _I64, _I64, _F, _P,
                           _I64, _I64, _I64, _I64, _P]),
    "h3q_gemm_i8_i32": (_I, [_P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _P]),
    "h3q_lora_down": (_I, [_P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _P]),
    "h3q_lora_down_workspace_bytes": (_I64, [_I64, _I64, _I64]),
    "h3q_lora_down_ws": (_I, [_P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _P, _I64, _P]),
    "h3q_rms_norm_modulate_quant": (_I, [_P, _I64, _P, _P, _P, _I64, _P, _I64, _I64, _F, _P, _I64, _I, _I, _P, _I64,
                                         _P, _P]),
    "h3q_residual_gate_rms_norm_modulate_quant": (_I, [_P, _I64, _P, _I64, _P, _P, _P, _P, _I64, _P, _I64, _I64, _F,
                                                       _P, _I64, _P, _I64, _I, _I, _P, _I64, _P, _P]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class H3QError(RuntimeError):
    """A native entry point returned a non-zero status."""


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH.name} is not built: run `python taomate-h3_amd/build.py` "
                    "(the quantized-linear path has no non-native fallback)"
                )
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _lib = handle
    return _lib


def call(name: str, *args) -> None:
    """Invoke an entry point and turn a non-zero status into H3QError."""
    handle = lib()
    status = getattr(handle, name)(*args)
    if status != 0:
        message = handle.h3q_last_error().decode(errors="replace")
        raise H3QError(f"{name} failed ({status}): {message}")
