"""FP8 quantizers of FL/inference/fused_kernels.py:771-820 on gfx950.

Same names, arguments and results as the reference; the Triton kernels
(amax partial/finalize + quantize, three launches) are replaced by
``h3q_quant_tensor_e4m3`` (two launches: partial maxima, then a pass that
folds them and quantizes).  Codes are bit-identical to the reference's eager
expression ``clamp(value / scale, +-448).to(float8_e4m3fn)``, whose quotient
is a bf16 tensor (bf16 divided by a 0-dim fp32 tensor), i.e. the binary32
quotient rounded to bf16 before the e4m3fn cast.

``quantize_fp8_e4m3_rowwise`` is the per-token (per-row) quantizer of the
per-token x per-channel FP8 W8A8 linear: fp32 quotient, scale
``max(amax_row / 448, 1e-12)``.  There is no bf16 fallback: inputs must be
bf16 tensors on a ROCm device.
"""

from __future__ import annotations

import torch

from .. import ops

FP8_MAX = 448.0


def _as_bf16(value: torch.Tensor, name: str) -> torch.Tensor:
    if value.dtype != torch.bfloat16:
        raise TypeError(f"{name} expects a bfloat16 tensor, got {value.dtype}")
    return value


def quantize_fp8_e4m3(value: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """Static per-tensor e4m3fn codes of ``value`` with the given fp32 scale
    (FL/inference/fused_kernels.py:771-785)."""
    _as_bf16(value, "quantize_fp8_e4m3")
    scale = scale.to(device=value.device, dtype=torch.float32)
    codes, _ = ops.quant_tensor_e4m3(value.contiguous(), scale.reshape(()))
    return codes


def quantize_fp8_e4m3_dynamic(value: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Dynamic per-tensor e4m3fn: (codes, 0-dim fp32 scale ``max(amax/448, 1e-12)``)
    (FL/inference/fused_kernels.py:788-820)."""
    _as_bf16(value, "quantize_fp8_e4m3_dynamic")
    return ops.quant_tensor_e4m3(value.contiguous())


def quantize_fp8_e4m3_rowwise(value: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Dynamic per-row e4m3fn of ``value [..., K]``: (codes [..., K], fp32 scales [..., 1])."""
    _as_bf16(value, "quantize_fp8_e4m3_rowwise")
    shape = value.shape
    flat = value.reshape(-1, int(shape[-1]))
    if flat.stride(-1) != 1:
        flat = flat.contiguous()
    codes, scales = ops.quant_rows(flat, ops.FMT_E4M3FN, ops.ROUND_DIV)
    return codes.reshape(shape), scales.reshape(*shape[:-1], 1)


__all__ = ["FP8_MAX", "quantize_fp8_e4m3", "quantize_fp8_e4m3_dynamic", "quantize_fp8_e4m3_rowwise"]
