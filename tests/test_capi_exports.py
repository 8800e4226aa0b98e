"""The C-ABI library loads on the CPU host and exports exactly the entry
points include/taomate_h3_amd.h declares (no compute calls: no GPU here)."""

from __future__ import annotations

import ctypes
import re
import subprocess

import pytest

from conftest import ROOT

HEADER = ROOT / "include" / "taomate_h3_amd.h"


def _declared() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(h3q_\w+)\s*\(", text, re.M))


def test_header_declares_entry_points():
    names = _declared()
    assert {"h3q_quant_rows", "h3q_quant_tensor_e4m3", "h3q_scaled_mm", "h3q_gemm_i8_i32",
            "h3q_lora_down", "h3q_lora_down_ws", "h3q_lora_down_workspace_bytes", "h3q_last_error", "h3q_version",
            "h3q_tiled_bytes", "h3q_quant_rows_tiled",
            "h3q_rms_norm_modulate_quant", "h3q_residual_gate_rms_norm_modulate_quant"} <= names


def test_library_exports_every_declared_symbol():
    from taomate_h3_amd import _lib

    if not _lib.LIB_PATH.exists():
        pytest.skip("library not built (run __graft_entry__.build())")
    handle = ctypes.CDLL(str(_lib.LIB_PATH))
    for name in _declared():
        assert hasattr(handle, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert exported == _declared(), exported ^ _declared()
    assert set(_lib.SIGNATURES) == _declared()


def test_version_and_error_without_gpu():
    from taomate_h3_amd import _lib

    if not _lib.LIB_PATH.exists():
        pytest.skip("library not built")
    lib = _lib.lib()
    assert lib.h3q_version() >= 200
    # Argument errors are rejected on the host before any launch.
    rc = lib.h3q_quant_rows(None, 4, 16, 16, 7, 0, None, 16, None, None)
    assert rc == 1
    assert b"unknown format" in lib.h3q_last_error()
    rc = lib.h3q_scaled_mm(0, None, 16, 0, None, 1, None, 16, 0, None, 1, None, None, 0, None, 0, 0, 1.0, None, 8,
                           4, 8, 24, None)
    assert rc == 1 and b"multiple of 16" in lib.h3q_last_error()
    # tiled operands: k must be a multiple of 128; tiled activations above 128
    # rows need the four-wave GEMM's shapes (k >= 256, 8-column stores)
    rc = lib.h3q_scaled_mm(0, None, 0, 0, None, 1, None, 0, 1, None, 1, None, None, 0, None, 0, 0, 1.0, None, 8,
                           4, 8, 64, None)
    assert rc == 1 and b"multiple of 128" in lib.h3q_last_error()
    rc = lib.h3q_scaled_mm(0, None, 0, 1, None, 1, None, 0, 1, None, 1, None, None, 0, None, 0, 0, 1.0, None, 8,
                           256, 8, 128, None)
    assert rc == 2 and b"tiled activations" in lib.h3q_last_error()
    rc = lib.h3q_scaled_mm(0, None, 0, 1, None, 1, None, 0, 1, None, 1, None, None, 0, None, 0, 0, 1.0, None, 12,
                           256, 12, 256, None)
    assert rc == 2 and b"tiled activations" in lib.h3q_last_error()
    # tiled activations take the LoRA epilogue only above 128 rows (the
    # four-wave GEMM); with 256 rows the call gets past that check
    p = ctypes.c_void_p(256)
    rc = lib.h3q_scaled_mm(0, None, 0, 1, None, 1, None, 0, 1, None, 1, None, p, 128, p, 128, 128, 1.0, None, 8,
                           64, 8, 256, None)
    assert rc == 2 and b"LoRA" in lib.h3q_last_error()
    rc = lib.h3q_scaled_mm(0, None, 0, 1, None, 1, None, 0, 1, None, 1, None, p, 128, p, 128, 128, 1.0, None, 8,
                           256, 8, 256, None)
    assert rc == 1 and b"null pointer" in lib.h3q_last_error()
    # 256 rows of a tiled operand must sit below a 32-bit offset: 256 * k < 2^31
    rc = lib.h3q_scaled_mm(0, None, 0, 1, None, 1, None, 0, 1, None, 1, None, None, 0, None, 0, 0, 1.0, None,
                           8, 4, 8, 1 << 23, None)
    assert rc == 2 and b"256 * k" in lib.h3q_last_error()
    # LoRA row strides above 8 MiB are refused
    rc = lib.h3q_scaled_mm(0, None, 128, 0, None, 1, None, 128, 0, None, 1, None, p, 1 << 22, p, 128, 128, 1.0,
                           None, 8, 4, 8, 128, None)
    assert rc == 2 and b"LoRA row stride" in lib.h3q_last_error()
    rc = lib.h3q_scaled_mm(0, None, 128, 5, None, 1, None, 128, 0, None, 1, None, None, 0, None, 0, 0, 1.0, None,
                           8, 4, 8, 128, None)
    assert rc == 1 and b"unknown operand layout" in lib.h3q_last_error()
    # binary16 output (format | H3Q_OUT_F16): not with LoRA, not with tiled activations above 128 rows
    f16 = 0x100
    rc = lib.h3q_scaled_mm(f16, None, 128, 0, None, 1, None, 128, 0, None, 1, None, p, 128, p, 128, 128, 1.0,
                           None, 8, 4, 8, 128, None)
    assert rc == 2 and b"bf16 only" in lib.h3q_last_error()
    rc = lib.h3q_scaled_mm(f16 | 1, None, 0, 1, None, 1, None, 0, 1, None, 1, None, None, 0, None, 0, 0, 1.0, None,
                           8, 256, 8, 256, None)
    assert rc == 2 and b"bf16 output" in lib.h3q_last_error()
    rc = lib.h3q_scaled_mm(0x200, None, 128, 0, None, 1, None, 128, 0, None, 1, None, None, 0, None, 0, 0, 1.0, None,
                           8, 4, 8, 128, None)
    assert rc == 1 and b"unknown format" in lib.h3q_last_error()
    # the typed per-tensor quantizer checks its dtype and form
    rc = lib.h3q_quant_tensor_e4m3_typed(None, 3, 0, 4, 16, 16, None, None, None, 16, None, None)
    assert rc == 1 and b"unknown input dtype" in lib.h3q_last_error()
    rc = lib.h3q_quant_tensor_e4m3_typed(None, 1, 2, 4, 16, 16, None, None, None, 16, None, None)
    assert rc == 1 and b"unknown quotient form" in lib.h3q_last_error()
    rc = lib.h3q_quant_rows_tiled(None, 4, 100, 100, 0, 0, 0, None, None, None)
    assert rc == 1 and b"multiple of 128" in lib.h3q_last_error()
    assert lib.h3q_tiled_bytes(17, 256) == 2 * 2 * 2048 and lib.h3q_tiled_bytes(16, 100) == 0


def test_norm_quant_errors_without_gpu():
    """The fused norm / modulate / quantize entry points reject bad requests
    on the host (no launch)."""
    from taomate_h3_amd import _lib

    if not _lib.LIB_PATH.exists():
        pytest.skip("library not built")
    lib = _lib.lib()
    f = ctypes.c_float(1e-6)
    # cols not a multiple of 8
    rc = lib.h3q_rms_norm_modulate_quant(None, 12, None, None, None, 12, None, 4, 12, f, None, 12, 1, 1, None, 12,
                                         None, None)
    assert rc == 2 and b"multiple of 8" in lib.h3q_last_error()
    # neither output nor codes
    rc = lib.h3q_rms_norm_modulate_quant(None, 16, None, None, None, 16, None, 4, 16, f, None, 16, 1, 1, None, 16,
                                         None, None)
    assert rc == 1 and b"neither" in lib.h3q_last_error()
    # e4m3 codes only in the division form
    rc = lib.h3q_residual_gate_rms_norm_modulate_quant(None, 16, None, 16, None, None, None, None, 16, None, 4, 16,
                                                       f, None, 16, None, 16, 0, 1, ctypes.c_void_p(64), 16,
                                                       ctypes.c_void_p(64), None)
    assert rc == 2 and b"division form" in lib.h3q_last_error()
    # width limit
    rc = lib.h3q_rms_norm_modulate_quant(None, 8200, None, None, None, 8200, None, 4, 8200, f, ctypes.c_void_p(64),
                                         8200, 1, 1, None, 8200, None, None)
    assert rc == 2 and b"above 8192" in lib.h3q_last_error()


def test_per_head_quant_errors_without_gpu():
    """h3q_quant_per_head_e4m3 validates its request on the host: empty
    reductions and too many heads are refused, an empty batch is a no-op."""
    from taomate_h3_amd import _lib

    if not _lib.LIB_PATH.exists():
        pytest.skip("library not built")
    lib = _lib.lib()
    p = ctypes.c_void_p(256)
    assert lib.h3q_quant_per_head_e4m3(p, 0, 16, 4, 128, p, p, p, None) == 0
    assert lib.h3q_quant_per_head_e4m3(p, 2, 16, 0, 128, p, p, p, None) == 0
    rc = lib.h3q_quant_per_head_e4m3(p, 1, 0, 4, 128, p, p, p, None)
    assert rc == 1 and b"empty" in lib.h3q_last_error()
    rc = lib.h3q_quant_per_head_e4m3(p, 1, 8, 4097, 8, p, p, p, None)
    assert rc == 2 and b"above 4096" in lib.h3q_last_error()
    rc = lib.h3q_quant_per_head_e4m3(p, 1, 8, 4, 128, None, p, p, None)
    assert rc == 1 and b"null" in lib.h3q_last_error()
    rc = lib.h3q_quant_per_head_e4m3(p, -1, 8, 4, 128, p, p, p, None)
    assert rc == 1 and b"negative" in lib.h3q_last_error()
    # workspace: batch * heads * chunks * column groups (up to 8 positions
    # per lane each), a chunk of at least 16 tokens, chunks * groups <= 1024
    assert lib.h3q_quant_per_head_workspace_floats(1, 8192, 40, 128) == 40 * 512 * 2
    assert lib.h3q_quant_per_head_workspace_floats(1, 65536, 56, 128) == 56 * 512 * 2
    assert lib.h3q_quant_per_head_workspace_floats(4, 65536, 8, 128) == 4 * 8 * 512
    assert lib.h3q_quant_per_head_workspace_floats(2, 3, 4096, 8) == 2 * 4096 * 8
    assert lib.h3q_quant_per_head_workspace_floats(1, 5, 3, 128) == 3


def test_ceilings_library_exports_measurement_entry_points():
    """bench.py's ceilings object loads its own measurement library (not the
    product's C ABI); it must be built and export its four entry points."""
    path = ROOT / "taomate-h3_amd" / "libh3q_ceilings.so"
    out = subprocess.run(["nm", "-D", "--defined-only", str(path)], capture_output=True, text=True).stdout
    names = set(re.findall(r"\bT (h3q_\w+)", out))
    assert names == {"h3q_ceil_read", "h3q_ceil_copy", "h3q_ceil_transform", "h3q_ceil_mfma"}
