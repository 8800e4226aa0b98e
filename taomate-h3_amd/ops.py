"""Tensor-level wrappers of the native entry points.

Each function checks dtypes, devices, shapes and strides on the host, raises
before any launch when they are wrong, and enqueues the kernels on the
current HIP stream of the input's device.  Output tensors may be supplied
(workspace reuse) or are allocated from torch's caching allocator.
"""

from __future__ import annotations

import ctypes
import weakref

import torch

from . import _lib

FMT_E4M3FN = 0
FMT_INT8 = 1
ROUND_DIV = 0
ROUND_RCP_MUL = 1
SCALE_PER_TENSOR = 0
SCALE_PER_ROW = 1
LAYOUT_ROWS = 0
LAYOUT_TILED = 1
OUT_F16 = 0x100      # scaled_mm format flag: binary16 output and bias
QUOTIENT_EAGER = 0   # per-tensor quotient forms of h3q_quant_tensor_e4m3_typed
QUOTIENT_TRITON = 1
SKINNY_MAX_M = 128   # rows up to which the weight-streaming GEMM runs

_CODE_DTYPES = {FMT_E4M3FN: torch.float8_e4m3fn, FMT_INT8: torch.int8}
_FORMATS = {torch.float8_e4m3fn: FMT_E4M3FN, torch.int8: FMT_INT8}


def _stream(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _ptr(t: torch.Tensor | None) -> ctypes.c_void_p | None:
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _require_gpu(name: str, *tensors: torch.Tensor | None) -> torch.device:
    device = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(f"{name}: tensors must be on a ROCm GPU, got {t.device}")
        if device is None:
            device = t.device
        elif t.device != device:
            raise RuntimeError(f"{name}: tensors on different devices ({device}, {t.device})")
    return device


def _rows_2d(name: str, t: torch.Tensor, dtype: torch.dtype) -> None:
    if t.dtype != dtype:
        raise TypeError(f"{name}: expected {dtype}, got {t.dtype}")
    if t.ndim != 2 or (t.shape[1] > 1 and t.stride(1) != 1):
        raise ValueError(f"{name}: expected a 2-D tensor with unit stride along the last dimension")


def code_dtype(fmt: int) -> torch.dtype:
    return _CODE_DTYPES[fmt]


def quant_rows(x: torch.Tensor, fmt: int, rounding: int = ROUND_DIV, *, codes: torch.Tensor | None = None,
               scales: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row quantization of bf16 ``x [rows, K]`` -> (codes [rows, K], scales [rows, 1] fp32)."""
    _require_gpu("quant_rows", x, codes, scales)
    _rows_2d("quant_rows x", x, torch.bfloat16)
    rows, cols = x.shape
    if codes is None:
        codes = torch.empty((rows, cols), device=x.device, dtype=_CODE_DTYPES[fmt])
    if scales is None:
        scales = torch.empty((rows, 1), device=x.device, dtype=torch.float32)
    _rows_2d("quant_rows codes", codes, _CODE_DTYPES[fmt])
    if tuple(codes.shape) != (rows, cols):
        raise ValueError(f"quant_rows: codes shape {tuple(codes.shape)} != {(rows, cols)}")
    if scales.dtype != torch.float32 or scales.numel() != rows or not scales.is_contiguous():
        raise ValueError("quant_rows: scales must be a contiguous fp32 tensor with one entry per row")
    _lib.call("h3q_quant_rows", _ptr(x), rows, cols, x.stride(0) if rows else cols, fmt, rounding, _ptr(codes),
              codes.stride(0) if rows else cols, _ptr(scales), _stream(x))
    return codes, scales


def _table(name: str, t: torch.Tensor, cols: int) -> int:
    """A [T, stride] bf16 modulation table (rows 16-byte aligned); returns its row stride."""
    _rows_2d(name, t, torch.bfloat16)
    if t.shape[1] != cols:
        raise ValueError(f"{name}: expected {cols} columns, got {t.shape[1]}")
    stride = t.stride(0) if t.shape[0] > 1 else cols
    if stride % 8:
        raise ValueError(f"{name}: row stride {stride} must be a multiple of 8 elements")
    return stride


def norm_modulate_quant(value: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor,
                        indices: torch.Tensor, eps: float, *, fmt: int | None = None, rounding: int = ROUND_DIV,
                        out: torch.Tensor | bool | None = None, codes: torch.Tensor | None = None,
                        scales: torch.Tensor | None = None, residual_gate: tuple | None = None):
    """RMSNorm + AdaLN modulate of bf16 rows, optionally preceded by the
    residual gate and followed by per-token quantization, in one kernel.

    ``value [rows, cols]`` (the residual when ``residual_gate=(branch, gate,
    hidden)`` is given: hidden = bf16(residual + bf16(gate[t] * branch)) is
    written into ``hidden``), ``weight [cols]``, ``scale``/``shift`` (and
    ``gate``) tables ``[T, cols]`` selected per row by int64 ``indices
    [rows]``.  ``out``: a bf16 tensor to receive the modulated rows, True to
    allocate one, None/False for none.  ``fmt``: code format for the per-token
    quantization (None: no codes).  Returns (out or None, codes or None,
    scales or None)."""
    branch = gate = hidden = None
    if residual_gate is not None:
        branch, gate, hidden = residual_gate
    want_out = out is True or isinstance(out, torch.Tensor)
    _require_gpu("norm_modulate_quant", value, weight, scale, shift, indices, branch, gate, hidden,
                 out if isinstance(out, torch.Tensor) else None, codes, scales)
    _rows_2d("norm_modulate_quant value", value, torch.bfloat16)
    rows, cols = value.shape
    if weight.dtype != torch.bfloat16 or weight.numel() != cols or not weight.is_contiguous():
        raise ValueError("norm_modulate_quant: weight must be a contiguous bf16 vector of the row width")
    stride = _table("norm_modulate_quant scale", scale, cols)
    if _table("norm_modulate_quant shift", shift, cols) != stride:
        raise ValueError("norm_modulate_quant: scale and shift tables differ in row stride")
    if indices.dtype != torch.int64 or indices.numel() != rows or not indices.is_contiguous():
        raise ValueError("norm_modulate_quant: indices must be a contiguous int64 tensor with one entry per row")
    if out is True:
        out = torch.empty((rows, cols), device=value.device, dtype=torch.bfloat16)
    elif not want_out:
        out = None
    if out is not None:
        _rows_2d("norm_modulate_quant out", out, torch.bfloat16)
        if tuple(out.shape) != (rows, cols):
            raise ValueError("norm_modulate_quant: out shape mismatch")
    if fmt is not None:
        if codes is None:
            codes = torch.empty((rows, cols), device=value.device, dtype=_CODE_DTYPES[fmt])
        if scales is None:
            scales = torch.empty((rows, 1), device=value.device, dtype=torch.float32)
        _rows_2d("norm_modulate_quant codes", codes, _CODE_DTYPES[fmt])
        if tuple(codes.shape) != (rows, cols):
            raise ValueError("norm_modulate_quant: codes shape mismatch")
        if scales.dtype != torch.float32 or scales.numel() != rows or not scales.is_contiguous():
            raise ValueError("norm_modulate_quant: scales must be a contiguous fp32 tensor with one entry per row")
    elif codes is not None or scales is not None:
        raise ValueError("norm_modulate_quant: codes / scales given without a format")
    if out is None and fmt is None:
        raise ValueError("norm_modulate_quant: neither a bf16 output nor codes requested")
    ld = lambda t: (t.stride(0) if rows > 1 else cols) if t is not None else cols
    common = (_ptr(weight), _ptr(scale), _ptr(shift), stride, _ptr(indices), rows, cols, float(eps))
    tail = (_ptr(out), ld(out), FMT_INT8 if fmt is None else fmt, rounding, _ptr(codes), ld(codes), _ptr(scales),
            _stream(value))
    if residual_gate is None:
        _lib.call("h3q_rms_norm_modulate_quant", _ptr(value), ld(value), *common, *tail)
    else:
        _rows_2d("norm_modulate_quant branch", branch, torch.bfloat16)
        _rows_2d("norm_modulate_quant hidden", hidden, torch.bfloat16)
        if tuple(branch.shape) != (rows, cols) or tuple(hidden.shape) != (rows, cols):
            raise ValueError("norm_modulate_quant: branch / hidden shape mismatch")
        if _table("norm_modulate_quant gate", gate, cols) != stride:
            raise ValueError("norm_modulate_quant: gate table row stride differs from scale / shift")
        _lib.call("h3q_residual_gate_rms_norm_modulate_quant", _ptr(value), ld(value), _ptr(branch), ld(branch),
                  _ptr(gate), *common, _ptr(hidden), ld(hidden), *tail)
    return out, codes, scales


def can_tile(rows: int, cols: int) -> bool:
    """Whether a [rows, cols] weight is stored tiled by the module mirror:
    the tiled matrix then has exactly the row-major shape and byte count."""
    return rows > 0 and rows % 16 == 0 and cols > 0 and cols % 128 == 0


# Storages that hold codes in the tiled layout.  The layout is a property of
# the bytes, so it is recorded against the storage: every view of a marked
# parameter -- ``weight.t()``, ``.data``, ``.detach()``, slices -- resolves to
# the same entry, for as long as any of them keeps the storage alive, while a
# copy (``.clone()``, ``.to()``, a new allocation at a reused address) does
# not.  An entry holds a weak reference to the storage object (torch keeps
# one Python object per live storage) and is dropped when that storage is
# freed; a lookup also checks that the storage found is the one recorded.
_TILED_STORAGES: dict[tuple[str, int, int], weakref.ref] = {}

# Module attribute set when this package stores the module's weight tiled.  A
# ``copy.deepcopy`` of the module copies the attribute with new, unmarked
# storage; ``module_weight_tiled`` re-marks such a copy.
TILED_WEIGHT_ATTR = "_h3q_tiled_weight"


def _storage_key(t: torch.Tensor) -> tuple[str, int, int]:
    st = t.untyped_storage()
    return (str(t.device), int(st.data_ptr()), int(st.nbytes()))


def _unmark(key: tuple[str, int, int], ref: weakref.ref) -> None:
    if _TILED_STORAGES.get(key) is ref:
        del _TILED_STORAGES[key]


def is_tiled(t: torch.Tensor | None) -> bool:
    """True when ``t`` (or any view of the same storage) holds tiled codes."""
    if t is None or not isinstance(t, torch.Tensor) or t.device.type == "meta":
        return False
    ref = _TILED_STORAGES.get(_storage_key(t))
    return ref is not None and ref() is t.untyped_storage()


def mark_tiled(t: torch.Tensor) -> torch.Tensor:
    """Record that the storage of the code tensor ``t`` holds the tiled layout
    (``t`` must cover its whole storage, as a freshly allocated weight does)."""
    if t.data_ptr() != t.untyped_storage().data_ptr() or t.numel() * t.element_size() != t.untyped_storage().nbytes():
        raise ValueError("mark_tiled: the tensor must cover its whole storage")
    if is_tiled(t):
        return t
    storage = t.untyped_storage()
    key = _storage_key(t)
    ref = weakref.ref(storage)
    _TILED_STORAGES[key] = ref
    weakref.finalize(storage, _unmark, key, ref)
    return t


def mark_module_weight_tiled(module: torch.nn.Module) -> torch.Tensor:
    """Mark ``module.weight``'s storage tiled and record the layout on the module."""
    mark_tiled(module.weight)
    setattr(module, TILED_WEIGHT_ATTR, True)
    return module.weight


def module_weight_tiled(module: torch.nn.Module) -> bool:
    """Whether ``module.weight`` holds tiled codes.  A weight whose module
    records the tiled layout but whose storage is unmarked is a copy of the
    tiled bytes (``copy.deepcopy`` of the module): its storage is marked
    here, so the copy computes what the original does.  deepcopy clones a
    parameter apart from the tensors that viewed it, so a precomputed
    ``_cutlass_w8a8_weight_t`` (H3/inference/w8a8.py:283) that no longer
    views the weight's storage is replaced by ``weight.t()``."""
    weight = getattr(module, "weight", None)
    if not is_tiled(weight):
        if not getattr(module, TILED_WEIGHT_ATTR, False) or not isinstance(weight, torch.Tensor):
            return False
        rows, cols = (int(v) for v in weight.shape) if weight.ndim == 2 else (0, 0)
        if weight.dtype not in (torch.int8, torch.float8_e4m3fn) or not can_tile(rows, cols):
            raise ValueError("the module records a tiled weight, but its weight is not a tiled code matrix")
        mark_tiled(weight)
    weight_t = getattr(module, "_cutlass_w8a8_weight_t", None)
    if isinstance(weight_t, torch.Tensor) and not is_tiled(weight_t):
        module._cutlass_w8a8_weight_t = weight.t()
    return True


def check_layout(name: str, t: torch.Tensor, tiled: bool) -> None:
    """Raise when a row-major call is made on a storage marked tiled."""
    if not tiled and is_tiled(t):
        raise ValueError(f"{name}: the operand's storage holds tiled codes; pass it with the tiled layout")


def quant_activations_for(x: torch.Tensor, fmt: int, rounding: int, weight: torch.Tensor, *,
                          codes: torch.Tensor | None = None, scales: torch.Tensor | None = None,
                          lora: bool = False):
    """Per-token quantization of the 2-D activations of a linear whose weight
    codes are ``weight`` (bf16 output): tiled when the weight is tiled and the
    GEMM reads tiled activations at this shape -- the weight-streaming GEMM
    for at most 128 tokens (no LoRA), the four-wave GEMM above that (K >= 256,
    N a multiple of 8, with or without the LoRA epilogue) -- else row-major.
    Returns (codes, scales, a_tiled); ``codes`` may be a larger workspace
    buffer of rows >= tiled_rows(m)."""
    m, k = x.shape
    n = int(weight.shape[0])
    four_wave = m > SKINNY_MAX_M and k >= 256 and n % 8 == 0
    fits = four_wave if lora else (0 < m <= SKINNY_MAX_M or four_wave)
    if is_tiled(weight) and k % 128 == 0 and fits:
        buf = None if codes is None else codes[:tiled_rows(m)]
        q, s = quant_rows_tiled(x, fmt, rounding, codes=buf, scales=scales)
        return q, s, True
    buf = None if codes is None else codes[:m]
    q, s = quant_rows(x, fmt, rounding, codes=buf, scales=scales)
    return q, s, False


def tiled_rows(rows: int) -> int:
    """Rows of storage a tiled operand of ``rows`` logical rows occupies (a multiple of 16)."""
    return (int(rows) + 15) // 16 * 16


def tiled_bytes(rows: int, cols: int) -> int:
    """Bytes of the tiled layout of a [rows, cols] code matrix (cols % 128 == 0), else 0."""
    return int(_lib.lib().h3q_tiled_bytes(int(rows), int(cols)))


def quant_rows_tiled(x: torch.Tensor, fmt: int, rounding: int = ROUND_DIV, *, codes: torch.Tensor | None = None,
                     row0: int = 0, scales: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row quantization of bf16 ``x [rows, K]`` into rows [row0, row0 + rows) of a tiled code matrix.

    ``codes`` is the whole tiled matrix, a contiguous [R, K] tensor of the code
    dtype with R a multiple of 16 (allocated here as [tiled_rows(rows), K]
    when omitted, which requires row0 == 0).  Scales are returned for the
    quantized rows only ([rows, 1] fp32)."""
    _require_gpu("quant_rows_tiled", x, codes, scales)
    _rows_2d("quant_rows_tiled x", x, torch.bfloat16)
    rows, cols = x.shape
    if cols % 128:
        raise ValueError(f"quant_rows_tiled: K={cols} must be a multiple of 128")
    if codes is None:
        if row0:
            raise ValueError("quant_rows_tiled: pass the tiled matrix when row0 > 0")
        codes = torch.empty((tiled_rows(rows), cols), device=x.device, dtype=_CODE_DTYPES[fmt])
    if codes.dtype != _CODE_DTYPES[fmt] or codes.ndim != 2 or codes.shape[1] != cols or not codes.is_contiguous():
        raise ValueError("quant_rows_tiled: codes must be a contiguous [R, K] tensor of the code dtype")
    if codes.shape[0] % 16 or row0 < 0 or row0 + rows > codes.shape[0]:
        raise ValueError(f"quant_rows_tiled: rows [{row0}, {row0 + rows}) do not fit a tiled matrix of "
                         f"{codes.shape[0]} rows (a multiple of 16)")
    if scales is None:
        scales = torch.empty((rows, 1), device=x.device, dtype=torch.float32)
    if scales.dtype != torch.float32 or scales.numel() != rows or not scales.is_contiguous():
        raise ValueError("quant_rows_tiled: scales must be a contiguous fp32 tensor with one entry per row")
    _lib.call("h3q_quant_rows_tiled", _ptr(x), rows, cols, x.stride(0) if rows else cols, fmt, rounding, int(row0),
              _ptr(codes), _ptr(scales), _stream(x))
    return codes, scales


_TENSOR_DTYPES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


def quant_tensor_e4m3(x: torch.Tensor, static_scale: torch.Tensor | None = None, *,
                      codes: torch.Tensor | None = None, scale: torch.Tensor | None = None,
                      workspace: torch.Tensor | None = None,
                      bf16_divisor: bool = False, eager: bool | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-tensor e4m3fn of a bf16, fp16 or fp32 tensor; returns (codes, 0-dim fp32 scale).

    ``eager``: torch's ``clamp(x / s, -448, 448)`` evaluated in x's dtype
    (the reference's eager expression on the GPU: for bf16 / fp16 input the
    divisor and the quotient are rounded to that dtype, for fp32 neither);
    otherwise the reference's Triton form, the fp32-divisor quotient rounded
    to bf16.  For bf16 input ``bf16_divisor`` is the older name of ``eager``."""
    _require_gpu("quant_tensor_e4m3", x, static_scale, codes, scale, workspace)
    if x.dtype not in _TENSOR_DTYPES:
        raise TypeError(f"quant_tensor_e4m3: expected bfloat16, float16 or float32 input, got {x.dtype}")
    if eager is None:
        eager = bf16_divisor
    shape = tuple(x.shape)
    x2 = x.reshape(-1, shape[-1]) if x.ndim != 2 else x
    if x2.ndim != 2 or x2.stride(-1) != 1:
        x2 = x2.contiguous()
    rows, cols = x2.shape
    if codes is None:
        codes = torch.empty(shape, device=x.device, dtype=torch.float8_e4m3fn)
    c2 = codes.view(rows, cols)
    if scale is None:
        scale = torch.empty((), device=x.device, dtype=torch.float32)
    if static_scale is not None:
        if static_scale.dtype != torch.float32 or static_scale.numel() != 1:
            raise TypeError("quant_tensor_e4m3: static scale must be one fp32 value")
        static_scale = static_scale.contiguous()
    elif workspace is None:
        n = int(_lib.lib().h3q_quant_tensor_workspace_floats(rows, cols))
        workspace = torch.empty(n, device=x.device, dtype=torch.float32)
    if x.dtype == torch.bfloat16:
        _lib.call("h3q_quant_tensor_e4m3_bf16_divisor" if eager else "h3q_quant_tensor_e4m3", _ptr(x2), rows,
                  cols, x2.stride(0), _ptr(static_scale), _ptr(workspace),
                  _ptr(c2), c2.stride(0), _ptr(scale), _stream(x))
    else:
        _lib.call("h3q_quant_tensor_e4m3_typed", _ptr(x2), _TENSOR_DTYPES[x.dtype], QUOTIENT_EAGER if eager
                  else QUOTIENT_TRITON, rows, cols, x2.stride(0), _ptr(static_scale), _ptr(workspace),
                  _ptr(c2), c2.stride(0), _ptr(scale), _stream(x))
    return codes, scale


def swiglu_quant(x: torch.Tensor, *, fmt: int | None = None, rounding: int = ROUND_DIV,
                 out: torch.Tensor | bool | None = None, codes: torch.Tensor | None = None,
                 scales: torch.Tensor | None = None):
    """Fused SwiGLU of bf16 rows ``x [rows, 2 * half]`` ([gate | up]):
    y = bf16(bf16(gate / (1 + exp(-gate))) * up), to ``out`` (a bf16 tensor,
    True to allocate one, None/False for none) and / or per-token codes in
    ``fmt`` (None: no codes).  Returns (out or None, codes or None, scales or None)."""
    want_out = out is True or isinstance(out, torch.Tensor)
    _require_gpu("swiglu_quant", x, out if isinstance(out, torch.Tensor) else None, codes, scales)
    _rows_2d("swiglu_quant x", x, torch.bfloat16)
    rows, width = x.shape
    if width % 2:
        raise ValueError(f"swiglu_quant: row width {width} is not [gate | up]")
    half = width // 2
    if out is True:
        out = torch.empty((rows, half), device=x.device, dtype=torch.bfloat16)
    elif not want_out:
        out = None
    if out is not None:
        _rows_2d("swiglu_quant out", out, torch.bfloat16)
        if tuple(out.shape) != (rows, half):
            raise ValueError("swiglu_quant: out shape mismatch")
    if fmt is not None:
        if codes is None:
            codes = torch.empty((rows, half), device=x.device, dtype=_CODE_DTYPES[fmt])
        if scales is None:
            scales = torch.empty((rows, 1), device=x.device, dtype=torch.float32)
        _rows_2d("swiglu_quant codes", codes, _CODE_DTYPES[fmt])
        if tuple(codes.shape) != (rows, half):
            raise ValueError("swiglu_quant: codes shape mismatch")
        if scales.dtype != torch.float32 or scales.numel() != rows or not scales.is_contiguous():
            raise ValueError("swiglu_quant: scales must be a contiguous fp32 tensor with one entry per row")
    elif codes is not None or scales is not None:
        raise ValueError("swiglu_quant: codes / scales given without a format")
    if out is None and fmt is None:
        raise ValueError("swiglu_quant: neither a bf16 output nor codes requested")
    ld = lambda t, w: (t.stride(0) if rows > 1 else w) if t is not None else w
    _lib.call("h3q_swiglu_quant", _ptr(x), ld(x, width), rows, half, _ptr(out), ld(out, half),
              FMT_INT8 if fmt is None else fmt, rounding, _ptr(codes), ld(codes, half), _ptr(scales), _stream(x))
    return out, codes, scales


def quant_per_head_e4m3(x: torch.Tensor, *, codes: torch.Tensor | None = None, scales: torch.Tensor | None = None,
                        workspace: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-(batch, head) e4m3fn of a bf16 ``x [B, S, H, D]``: (codes [B, S, H, D]
    float8_e4m3fn, scales [B, H] fp32) with scale = max(amax * RN(1/448), 1e-12)
    over (S, D) and an fp32 quotient."""
    _require_gpu("quant_per_head_e4m3", x, codes, scales, workspace)
    if x.dtype != torch.bfloat16:
        raise TypeError(f"quant_per_head_e4m3: expected bfloat16 input, got {x.dtype}")
    if x.ndim != 4:
        raise ValueError(f"quant_per_head_e4m3: expected [batch, seq, heads, head_dim], got shape {tuple(x.shape)}")
    x = x.contiguous()
    b, s, h, d = (int(v) for v in x.shape)
    if codes is None:
        codes = torch.empty(x.shape, device=x.device, dtype=torch.float8_e4m3fn)
    if codes.shape != x.shape or codes.dtype != torch.float8_e4m3fn or not codes.is_contiguous():
        raise ValueError("quant_per_head_e4m3: codes must be a contiguous float8_e4m3fn tensor of the input shape")
    if scales is None:
        scales = torch.empty((b, h), device=x.device, dtype=torch.float32)
    if scales.numel() != b * h or scales.dtype != torch.float32 or not scales.is_contiguous():
        raise ValueError("quant_per_head_e4m3: scales must be a contiguous fp32 tensor of batch x heads entries")
    if workspace is None:
        n = int(_lib.lib().h3q_quant_per_head_workspace_floats(b, s, h, d))
        workspace = torch.empty(n, device=x.device, dtype=torch.float32)
    _lib.call("h3q_quant_per_head_e4m3", _ptr(x), b, s, h, d, _ptr(workspace), _ptr(codes), _ptr(scales),
              _stream(x))
    return codes, scales


def _scale_kind(name: str, s: torch.Tensor, count: int) -> int:
    if s.dtype != torch.float32:
        raise TypeError(f"{name}: scales must be fp32, got {s.dtype}")
    if not s.is_contiguous():
        raise ValueError(f"{name}: scales must be contiguous")
    if s.numel() == 1 and count != 1:
        return SCALE_PER_TENSOR
    if s.numel() == count:
        return SCALE_PER_ROW
    raise ValueError(f"{name}: {s.numel()} scales for {count} rows")


def scaled_mm(a: torch.Tensor, b: torch.Tensor, a_scale: torch.Tensor, b_scale: torch.Tensor, *,
              bias: torch.Tensor | None = None, lora_t: torch.Tensor | None = None,
              lora_b: torch.Tensor | None = None, lora_scale: float = 1.0,
              out: torch.Tensor | None = None, a_tiled: bool = False, b_tiled: bool = False,
              m: int | None = None, n: int | None = None,
              out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """out[m, n] = a_scale[m] * (b_scale[n] * (a @ b^T)) [+ bias] [+ lora_scale * lora_t @ lora_b^T],
    rounded once to ``out_dtype`` (bf16, or float16 as torch._scaled_mm's
    out_dtype; the bias is then float16 too).

    ``a`` [m, k] and ``b`` [n, k] are both e4m3fn or both int8 codes (``b`` in
    the nn.Linear [out, in] layout).  A tiled operand (``a_tiled`` /
    ``b_tiled``, see quant_rows_tiled) is a contiguous [R, k] tensor with R the
    row count rounded up to 16; ``m`` / ``n`` give the logical row counts when
    they differ from R."""
    _require_gpu("scaled_mm", a, b, a_scale, b_scale, bias, lora_t, lora_b, out)
    if a.dtype not in _FORMATS or b.dtype != a.dtype:
        raise TypeError(f"scaled_mm: operands must both be e4m3fn or int8, got {a.dtype} and {b.dtype}")
    _rows_2d("scaled_mm a", a, a.dtype)
    _rows_2d("scaled_mm b", b, b.dtype)
    k = a.shape[1]
    m = a.shape[0] if m is None else int(m)
    n = b.shape[0] if n is None else int(n)
    for name, t, rows, tiled in (("a", a, m, a_tiled), ("b", b, n, b_tiled)):
        need = tiled_rows(rows) if tiled else rows
        if t.shape[0] < need or (tiled and not t.is_contiguous()):
            raise ValueError(f"scaled_mm: {name} holds {t.shape[0]} rows, {need} needed"
                             + (" (tiled operands are contiguous, rows rounded up to 16)" if tiled else ""))
    if b.shape[1] != k:
        raise ValueError(f"scaled_mm: inner dimensions differ ({k} vs {b.shape[1]})")
    check_layout("scaled_mm a", a, a_tiled)
    check_layout("scaled_mm b", b, b_tiled)
    ak = _scale_kind("scaled_mm a_scale", a_scale, m)
    bk = _scale_kind("scaled_mm b_scale", b_scale, n)
    if out_dtype not in (torch.bfloat16, torch.float16):
        raise TypeError(f"scaled_mm: out_dtype must be bfloat16 or float16, got {out_dtype}")
    if bias is not None:
        if bias.dtype != out_dtype or bias.numel() != n or not bias.is_contiguous():
            raise ValueError(f"scaled_mm: bias must be a contiguous {out_dtype} vector of length n")
    rank = 0
    if (lora_t is None) != (lora_b is None):
        raise ValueError("scaled_mm: lora_t and lora_b go together")
    if lora_t is not None:
        _rows_2d("scaled_mm lora_t", lora_t, torch.bfloat16)
        _rows_2d("scaled_mm lora_b", lora_b, torch.bfloat16)
        rank = lora_t.shape[1]
        if lora_t.shape[0] != m or tuple(lora_b.shape) != (n, rank):
            raise ValueError("scaled_mm: LoRA shapes must be t [m, r] and B [n, r]")
    if out is None:
        out = torch.empty((m, n), device=a.device, dtype=out_dtype)
    _rows_2d("scaled_mm out", out, out_dtype)
    if tuple(out.shape) != (m, n):
        raise ValueError(f"scaled_mm: out shape {tuple(out.shape)} != {(m, n)}")
    if m == 0 or n == 0:
        return out
    fmt = _FORMATS[a.dtype] | (OUT_F16 if out_dtype == torch.float16 else 0)
    _lib.call("h3q_scaled_mm", fmt, _ptr(a), a.stride(0), LAYOUT_TILED if a_tiled else LAYOUT_ROWS,
              _ptr(a_scale), ak, _ptr(b), b.stride(0), LAYOUT_TILED if b_tiled else LAYOUT_ROWS, _ptr(b_scale), bk,
              _ptr(bias), _ptr(lora_t), lora_t.stride(0) if lora_t is not None else 0,
              _ptr(lora_b), lora_b.stride(0) if lora_b is not None else 0, rank, float(lora_scale), _ptr(out),
              out.stride(0), m, n, k, _stream(a))
    return out


def gemm_i8_i32(a: torch.Tensor, b: torch.Tensor, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """Exact int32 accumulators a @ b^T of int8 a [m, k], b [n, k]."""
    _require_gpu("gemm_i8_i32", a, b, out)
    _rows_2d("gemm_i8_i32 a", a, torch.int8)
    _rows_2d("gemm_i8_i32 b", b, torch.int8)
    m, k = a.shape
    n = b.shape[0]
    if b.shape[1] != k:
        raise ValueError("gemm_i8_i32: inner dimensions differ")
    if out is None:
        out = torch.empty((m, n), device=a.device, dtype=torch.int32)
    _rows_2d("gemm_i8_i32 out", out, torch.int32)
    if m == 0 or n == 0:
        return out
    _lib.call("h3q_gemm_i8_i32", _ptr(a), a.stride(0), _ptr(b), b.stride(0), _ptr(out), out.stride(0), m, n, k,
              _stream(a))
    return out


def lora_down(x: torch.Tensor, lora_a: torch.Tensor, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """t = bf16(x @ lora_a^T) for bf16 x [m, k], lora_a [r, k]."""
    _require_gpu("lora_down", x, lora_a, out)
    _rows_2d("lora_down x", x, torch.bfloat16)
    _rows_2d("lora_down lora_a", lora_a, torch.bfloat16)
    m, k = x.shape
    rank = lora_a.shape[0]
    if lora_a.shape[1] != k:
        raise ValueError("lora_down: inner dimensions differ")
    if out is None:
        out = torch.empty((m, rank), device=x.device, dtype=torch.bfloat16)
    _rows_2d("lora_down out", out, torch.bfloat16)
    if m == 0:
        return out
    # Few rows: the library splits K and needs a binary32 workspace for the
    # slices' partial sums (allocated here, so graph capture keeps it).
    ws_bytes = int(_lib.lib().h3q_lora_down_workspace_bytes(m, k, rank))
    if ws_bytes == 0:
        _lib.call("h3q_lora_down", _ptr(x), x.stride(0), _ptr(lora_a), lora_a.stride(0), _ptr(out), out.stride(0), m,
                  k, rank, _stream(x))
        return out
    ws = torch.empty(ws_bytes, device=x.device, dtype=torch.uint8)
    _lib.call("h3q_lora_down_ws", _ptr(x), x.stride(0), _ptr(lora_a), lora_a.stride(0), _ptr(out), out.stride(0), m,
              k, rank, _ptr(ws), ws_bytes, _stream(x))
    return out
