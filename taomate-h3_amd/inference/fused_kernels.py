"""FP8 quantizers of FL/inference/fused_kernels.py:771-877 and the
RMSNorm/AdaLN producers of H3/inference/fused_kernels.py:700-773 on gfx950.

Same names, arguments and results as the reference; the Triton kernels
(amax partial/finalize + quantize, three launches) are replaced by
``h3q_quant_tensor_e4m3`` (two launches: partial maxima, then a pass that
folds them and quantizes).  The quotient is a bf16 tensor (bf16 divided by a
0-dim fp32 tensor), i.e. the binary32 quotient rounded to bf16 before the
e4m3fn cast.  Its divisor follows the reference's mode: after
``enable_h3_inference_fused_kernels()`` the fp32 scale (the Triton kernel's
``_round_bf16(div_rn(value, scale))``), otherwise the scale rounded to bf16
(the eager ``clamp(value / scale, +-448)`` as torch computes it on the GPU).

Dynamic scales are ``max(amax * RN(1/448), 1e-12)``: the reference's
``clamp(amax / 448, min=1e-12)`` as torch evaluates it on the GPU (a tensor
divided by a Python scalar is a multiply by the binary32 reciprocal) and as its
Triton finalize kernels write it.

``quantize_fp8_e4m3_per_head`` (``h3q_quant_per_head_e4m3``) keeps the
reference's per-(batch, head) scales and fp32 quotient for the FP8 attention
operands.  ``quantize_fp8_e4m3_rowwise`` is the per-token (per-row) quantizer
of the per-token x per-channel FP8 W8A8 linear: fp32 quotient.  There is no
bf16 fallback: inputs must be bf16 tensors on a ROCm device.

``fused_rms_norm_modulate`` and ``fused_residual_gate_rms_norm_modulate``
keep the reference's names, arguments, results and index check.  Their
``*_w8a8`` variants run the same kernel with the per-token activation
quantizer of the next W8A8 linear folded in and return a
``QuantizedActivations`` that ``cutlass_w8a8_linear`` accepts in place of the
bf16 input, so the QKV / fc1 input is never written and re-read in bf16.  The
sum of squares and rsqrt are computed in a fixed order with IEEE operations
(the reference's Triton kernels use an approximate rsqrt); see
include/taomate_h3_amd.h.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .. import ops

FP8_MAX = 448.0
_ENABLED = False


def enable_h3_inference_fused_kernels() -> None:
    """FL/inference/fused_kernels.py:14-18: select the reference's Triton forms.
    The one observable difference on this path is the per-tensor FP8 quotient:
    enabled, the fp32 scale divides (the Triton kernel); disabled, the divisor
    is the scale rounded to bf16, as the reference's eager expression
    evaluates on the GPU.  The per-head quantizer is the same either way."""
    global _ENABLED
    _ENABLED = True


def enable_h3_sol_engine_fusions() -> None:
    """FL/inference/fused_kernels.py:21-26 (implies the fused kernels)."""
    enable_h3_inference_fused_kernels()


def h3_inference_fused_kernels_enabled() -> bool:
    return _ENABLED


def _as_bf16(value: torch.Tensor, name: str) -> torch.Tensor:
    if value.dtype != torch.bfloat16:
        raise TypeError(f"{name} expects a bfloat16 tensor, got {value.dtype}")
    return value


def quantize_fp8_e4m3(value: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """Static per-tensor e4m3fn codes of a bf16, fp16 or fp32 ``value`` with
    the given fp32 scale (FL/inference/fused_kernels.py:771-785): the eager
    expression in value's dtype until the fused kernels are enabled, then
    the Triton kernel's bf16-rounded fp32 quotient."""
    scale = scale.to(device=value.device, dtype=torch.float32)
    codes, _ = ops.quant_tensor_e4m3(value.contiguous(), scale.reshape(()), eager=not _ENABLED)
    return codes


def quantize_fp8_e4m3_dynamic(value: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Dynamic per-tensor e4m3fn of a bf16, fp16 or fp32 tensor: (codes, 0-dim
    fp32 scale ``max(amax * RN(1/448), 1e-12)``) (FL/inference/fused_kernels.py:788-820)."""
    return ops.quant_tensor_e4m3(value.contiguous(), eager=not _ENABLED)


def quantize_fp8_e4m3_per_head(value: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-(batch, head) e4m3fn of attention operands ``value [B, S, H, D]``
    (FL/inference/fused_kernels.py:823-877): (codes [B, S, H, D], fp32 scales
    [B, H]), the scales being the descales FlashAttention-3 takes
    (FL/streaming/attention_hook.py:1018-1043, FL/streaming/cache.py:838-853)."""
    _as_bf16(value, "quantize_fp8_e4m3_per_head")
    return ops.quant_per_head_e4m3(value)


def quantize_fp8_e4m3_rowwise(value: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Dynamic per-row e4m3fn of ``value [..., K]``: (codes [..., K], fp32 scales [..., 1])."""
    _as_bf16(value, "quantize_fp8_e4m3_rowwise")
    shape = value.shape
    flat = value.reshape(-1, int(shape[-1]))
    if flat.stride(-1) != 1:
        flat = flat.contiguous()
    codes, scales = ops.quant_rows(flat, ops.FMT_E4M3FN, ops.ROUND_DIV)
    return codes.reshape(shape), scales.reshape(*shape[:-1], 1)


def fused_swiglu(value: torch.Tensor) -> torch.Tensor:
    """SwiGLU of ``value [..., 2F]`` ([gate | up]) -> ``[..., F]`` bf16
    (H3/inference/fused_kernels.py:663-677; the eager F.silu(gate) * up of
    H3/model/layers.py:476-479): bf16(bf16(gate / (1 + exp(-gate))) * up)."""
    _as_bf16(value, "fused_swiglu")
    shape = value.shape
    flat = value.reshape(-1, int(shape[-1]))
    if flat.stride(-1) != 1 or flat.data_ptr() % 16 or (flat.shape[0] > 1 and flat.stride(0) % 8):
        flat = flat.contiguous()
    out, _, _ = ops.swiglu_quant(flat, out=True)
    return out.reshape(*shape[:-1], int(shape[-1]) // 2)


def fused_swiglu_w8a8(value: torch.Tensor, *, fmt: int = ops.FMT_INT8,
                      keep_dense: bool = False) -> QuantizedActivations:
    """``fused_swiglu`` with the per-token quantizer of the fc2 W8A8 linear
    folded in (int8 in vLLM's form, or e4m3fn): the fc2 input is never
    written and re-read in bf16 (unless ``keep_dense``)."""
    _as_bf16(value, "fused_swiglu_w8a8")
    shape = value.shape
    flat = value.reshape(-1, int(shape[-1]))
    if flat.stride(-1) != 1 or flat.data_ptr() % 16 or (flat.shape[0] > 1 and flat.stride(0) % 8):
        flat = flat.contiguous()
    rounding = ops.ROUND_RCP_MUL if fmt == ops.FMT_INT8 else ops.ROUND_DIV
    dense, codes, scales = ops.swiglu_quant(flat, fmt=fmt, rounding=rounding, out=keep_dense)
    out_shape = (*shape[:-1], int(shape[-1]) // 2)
    return QuantizedActivations(codes, scales, out_shape, fmt,
                                None if dense is None else dense.reshape(out_shape))


@dataclass
class QuantizedActivations:
    """Per-token codes of a linear's input: ``codes [M, K]`` (row-major),
    ``scales [M, 1]`` fp32, the activation ``shape [..., K]`` they stand for,
    the code format, and optionally the bf16 rows themselves (``dense``, for a
    LoRA side branch that needs them)."""

    codes: torch.Tensor
    scales: torch.Tensor
    shape: tuple
    fmt: int = ops.FMT_INT8
    dense: torch.Tensor | None = None


def as_dense(inputs):
    """The bf16 activations behind ``inputs`` (a tensor, or a
    QuantizedActivations produced with ``keep_dense=True``)."""
    if not isinstance(inputs, QuantizedActivations):
        return inputs
    if inputs.dense is None:
        raise TypeError("this linear needs the bf16 activations; produce them with keep_dense=True")
    return inputs.dense.reshape(inputs.shape)


def _modulation_inputs(value: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor, indices: torch.Tensor,
                       what: str):
    flat = value.reshape(-1, int(value.shape[-1]))
    if flat.stride(-1) != 1 or (flat.shape[0] > 1 and flat.stride(0) % 8):
        flat = flat.contiguous()
    index = indices.reshape(-1)
    if int(index.numel()) != int(flat.shape[0]):
        raise ValueError(f"SOL {what} indices do not cover every row")
    index = index.to(torch.int64).contiguous()
    if scale.stride(-1) != 1 or shift.stride(-1) != 1:
        scale, shift = scale.contiguous(), shift.contiguous()
    return flat, index, scale, shift


def fused_rms_norm_modulate(value: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor,
                            indices: torch.Tensor, eps: float) -> torch.Tensor:
    """bf16(bf16(RMSNorm(value) * bf16(1 + scale[idx])) + shift[idx])
    (H3/inference/fused_kernels.py:700-730)."""
    _as_bf16(value, "fused_rms_norm_modulate")
    flat, index, scale, shift = _modulation_inputs(value, scale, shift, indices, "RMSNorm/AdaLN")
    out, _, _ = ops.norm_modulate_quant(flat, weight.contiguous(), scale, shift, index, eps, out=True)
    return out.reshape(value.shape)


def fused_residual_gate_rms_norm_modulate(residual: torch.Tensor, branch: torch.Tensor, gate: torch.Tensor,
                                          weight: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor,
                                          indices: torch.Tensor, eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """(hidden, output): hidden = bf16(residual + bf16(gate[idx] * branch)),
    output = the modulated RMSNorm of hidden (H3/inference/fused_kernels.py:733-773)."""
    _as_bf16(residual, "fused_residual_gate_rms_norm_modulate")
    flat, index, scale, shift = _modulation_inputs(residual, scale, shift, indices, "residual/AdaLN")
    branch_flat = branch.reshape(-1, int(branch.shape[-1])).contiguous()
    gate = gate.contiguous() if gate.stride(-1) != 1 else gate
    hidden = torch.empty_like(flat)
    out, _, _ = ops.norm_modulate_quant(flat, weight.contiguous(), scale, shift, index, eps, out=True,
                                        residual_gate=(branch_flat, gate, hidden))
    return hidden.reshape(residual.shape), out.reshape(residual.shape)


def fused_rms_norm_modulate_w8a8(value: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor,
                                 shift: torch.Tensor, indices: torch.Tensor, eps: float, *,
                                 fmt: int = ops.FMT_INT8, keep_dense: bool = False) -> QuantizedActivations:
    """``fused_rms_norm_modulate`` whose output goes straight into per-token
    codes for the next W8A8 linear (int8 in the vLLM form, or e4m3fn)."""
    _as_bf16(value, "fused_rms_norm_modulate_w8a8")
    flat, index, scale, shift = _modulation_inputs(value, scale, shift, indices, "RMSNorm/AdaLN")
    rounding = ops.ROUND_RCP_MUL if fmt == ops.FMT_INT8 else ops.ROUND_DIV
    dense, codes, scales = ops.norm_modulate_quant(flat, weight.contiguous(), scale, shift, index, eps,
                                                   fmt=fmt, rounding=rounding, out=bool(keep_dense))
    return QuantizedActivations(codes, scales, tuple(value.shape), fmt, dense)


def fused_residual_gate_rms_norm_modulate_w8a8(residual: torch.Tensor, branch: torch.Tensor, gate: torch.Tensor,
                                               weight: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor,
                                               indices: torch.Tensor, eps: float, *, fmt: int = ops.FMT_INT8,
                                               keep_dense: bool = False
                                               ) -> tuple[torch.Tensor, QuantizedActivations]:
    """``fused_residual_gate_rms_norm_modulate`` with the modulated output
    quantized per token: (hidden, QuantizedActivations)."""
    _as_bf16(residual, "fused_residual_gate_rms_norm_modulate_w8a8")
    flat, index, scale, shift = _modulation_inputs(residual, scale, shift, indices, "residual/AdaLN")
    branch_flat = branch.reshape(-1, int(branch.shape[-1])).contiguous()
    gate = gate.contiguous() if gate.stride(-1) != 1 else gate
    hidden = torch.empty_like(flat)
    rounding = ops.ROUND_RCP_MUL if fmt == ops.FMT_INT8 else ops.ROUND_DIV
    dense, codes, scales = ops.norm_modulate_quant(flat, weight.contiguous(), scale, shift, index, eps, fmt=fmt,
                                                   rounding=rounding, out=bool(keep_dense),
                                                   residual_gate=(branch_flat, gate, hidden))
    return hidden.reshape(residual.shape), QuantizedActivations(codes, scales, tuple(residual.shape), fmt, dense)


__all__ = ["FP8_MAX", "QuantizedActivations", "as_dense", "enable_h3_inference_fused_kernels",
           "enable_h3_sol_engine_fusions", "fused_residual_gate_rms_norm_modulate", "fused_swiglu",
           "fused_swiglu_w8a8", "h3_inference_fused_kernels_enabled",
           "fused_residual_gate_rms_norm_modulate_w8a8", "fused_rms_norm_modulate", "fused_rms_norm_modulate_w8a8",
           "quantize_fp8_e4m3", "quantize_fp8_e4m3_dynamic", "quantize_fp8_e4m3_per_head",
           "quantize_fp8_e4m3_rowwise"]
