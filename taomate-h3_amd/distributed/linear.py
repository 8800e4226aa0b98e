"""The quantized-linear dispatch of the parallel linear layers.

Drop-in for the quantized-linear seam of H3/distributed/linear.py:15-191 and
FL/distributed/linear.py:16-181:

* ``_module_linear(module, inputs, bias)`` (H3/distributed/linear.py:15-33)
  dispatches on module attributes: ``_cutlass_w8a8_weight_scale`` -> int8
  W8A8, ``_fp8_w8a8_weight_scale`` -> per-token x per-channel FP8 W8A8 (the
  BASELINE.json format; no counterpart in the reference), ``_fp8_weight_scale`` ->
  per-tensor FP8 (FL), otherwise ``F.linear``.
* ``_linear(...)`` keeps FL's functional signature (FL/distributed/linear.py:50-101)
  including the "cannot combine" error.
* ``_module_fp8_input_scale`` and the two context managers keep FL's
  calibrated-scale protocol (FL/distributed/linear.py:16-47,104-128).

The parallel linear layers themselves (ColumnParallelLinear,
MergedColumnParallelLinear, RowParallelLinear) stay the reference's: their
forward calls ``_module_linear``, which this module replaces.  This build runs
on one GPU; steps that exchange data across tensor-parallel ranks raise
``NotImplementedError`` (``_cross_rank``).
"""

from __future__ import annotations

from collections.abc import Iterator
from contextlib import contextmanager
from contextvars import ContextVar

import torch
import torch.nn as nn
import torch.nn.functional as F

from .. import ops


def _cross_rank(what: str) -> NotImplementedError:
    return NotImplementedError(f"{what} across tensor-parallel ranks is not part of this single-GPU build")


# ------------------------------------------------------------------ dispatch

def _fp8_w8a8_linear(inputs: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor,
                     bias: torch.Tensor | None) -> torch.Tensor:
    """Per-token dynamic e4m3fn activations x per-channel e4m3fn weights
    (the activations may come pre-quantized from a fused producer)."""
    from ..inference.fused_kernels import QuantizedActivations

    shape = (*inputs.shape[:-1], int(weight.shape[0]))
    if isinstance(inputs, QuantizedActivations):
        if inputs.fmt != ops.FMT_E4M3FN:
            raise TypeError("FP8 W8A8 linear expects e4m3fn activation codes")
        out = ops.scaled_mm(inputs.codes, weight, inputs.scales.reshape(-1), weight_scale.reshape(-1), bias=bias,
                            b_tiled=ops.is_tiled(weight), m=int(inputs.codes.shape[0]))
        return out.reshape(shape)
    flat = inputs.reshape(-1, int(inputs.shape[-1])).contiguous()
    q, s, a_tiled = ops.quant_activations_for(flat, ops.FMT_E4M3FN, ops.ROUND_DIV, weight)
    out = ops.scaled_mm(q, weight, s.reshape(-1), weight_scale.reshape(-1), bias=bias, a_tiled=a_tiled,
                        b_tiled=ops.is_tiled(weight), m=int(flat.shape[0]))
    return out.reshape(shape)


def _fp8_tensor_linear(inputs: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor,
                       bias: torch.Tensor | None, input_scale: torch.Tensor | None) -> torch.Tensor:
    """Per-tensor FP8 (FL/distributed/linear.py:80-101): dynamic or static
    activation scale, then the scaled GEMM in place of torch._scaled_mm."""
    from ..inference.fused_kernels import quantize_fp8_e4m3, quantize_fp8_e4m3_dynamic

    shape = (*inputs.shape[:-1], int(weight.shape[0]))
    flat = inputs.reshape(-1, int(inputs.shape[-1]))
    if input_scale is None:
        q, input_scale = quantize_fp8_e4m3_dynamic(flat)
    else:
        q = quantize_fp8_e4m3(flat, input_scale)
    if bias is not None and bias.dtype != torch.bfloat16:
        bias = bias.to(torch.bfloat16)
    out = ops.scaled_mm(q, weight, input_scale.reshape(1).to(torch.float32),
                        weight_scale.reshape(1).to(torch.float32), bias=bias)
    return out.reshape(shape)


def _module_linear(module: nn.Module, inputs: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
    """H3/distributed/linear.py:15-33 plus the FP8 formats.  ``inputs`` may
    also be per-token codes from a fused producer (QuantizedActivations): the
    per-token W8A8 paths consume them directly, the others use their bf16 rows."""
    from ..inference.fused_kernels import QuantizedActivations, as_dense

    if getattr(module, ops.TILED_WEIGHT_ATTR, False):
        ops.module_weight_tiled(module)  # re-marks the storage of a deep-copied tiled weight
    scale = getattr(module, "_cutlass_w8a8_weight_scale", None)
    if isinstance(inputs, QuantizedActivations) and scale is None and \
            getattr(module, "_fp8_w8a8_weight_scale", None) is None:
        inputs = as_dense(inputs)
    if scale is not None:
        from ..inference.w8a8 import cutlass_w8a8_linear

        return cutlass_w8a8_linear(
            inputs,
            module.weight,
            scale,
            bias=bias,
            workspace=getattr(module, "_cutlass_w8a8_workspace", None),
            weight_t=getattr(module, "_cutlass_w8a8_weight_t", None),
            weight_scale_t=getattr(module, "_cutlass_w8a8_weight_scale_t", None),
        )
    fp8_rows = getattr(module, "_fp8_w8a8_weight_scale", None)
    if fp8_rows is not None:
        return _fp8_w8a8_linear(inputs, module.weight, fp8_rows, bias)
    fp8_tensor = getattr(module, "_fp8_weight_scale", None)
    if fp8_tensor is not None:
        return _fp8_tensor_linear(inputs, module.weight, fp8_tensor, bias, _module_fp8_input_scale(module, inputs))
    return F.linear(inputs, module.weight, bias)


def _linear(inputs: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None,
            fp8_weight_scale: torch.Tensor | None, fp8_input_scale: torch.Tensor | None = None,
            cutlass_w8a8_weight_scale: torch.Tensor | None = None, cutlass_w8a8_workspace: object | None = None,
            cutlass_w8a8_weight_t: torch.Tensor | None = None,
            cutlass_w8a8_weight_scale_t: torch.Tensor | None = None) -> torch.Tensor:
    """FL/distributed/linear.py:50-101."""
    if cutlass_w8a8_weight_scale is not None:
        if fp8_weight_scale is not None:
            raise RuntimeError("a linear cannot combine CUTLASS W8A8 with another quantizer")
        from ..inference.w8a8 import cutlass_w8a8_linear

        return cutlass_w8a8_linear(inputs, weight, cutlass_w8a8_weight_scale, bias=bias,
                                   workspace=cutlass_w8a8_workspace, weight_t=cutlass_w8a8_weight_t,
                                   weight_scale_t=cutlass_w8a8_weight_scale_t)
    if fp8_weight_scale is None:
        return F.linear(inputs, weight, bias)
    return _fp8_tensor_linear(inputs, weight, fp8_weight_scale, bias, fp8_input_scale)


# ------------------------------------------------ calibrated FP8 input scale

_FP8_ACTIVATION_SCALE_POLICY: ContextVar[str] = ContextVar("taomate_h3_amd_fp8_activation_scale_policy",
                                                           default="current")
_FP8_ACTIVATION_CALIBRATION_SUSPENDED: ContextVar[bool] = ContextVar(
    "taomate_h3_amd_fp8_activation_calibration_suspended", default=False)


@contextmanager
def use_fp8_activation_scale_policy(policy: str) -> Iterator[None]:
    """Select local-current or cross-stage-shared calibrated FP8 scales."""
    if policy not in {"current", "prefix_shared"}:
        raise ValueError("unsupported FP8 activation scale policy")
    token = _FP8_ACTIVATION_SCALE_POLICY.set(policy)
    try:
        yield
    finally:
        _FP8_ACTIVATION_SCALE_POLICY.reset(token)


@contextmanager
def suspend_fp8_activation_calibration() -> Iterator[None]:
    """Run FP8 with per-forward scales without consuming calibration samples."""
    token = _FP8_ACTIVATION_CALIBRATION_SUSPENDED.set(True)
    try:
        yield
    finally:
        _FP8_ACTIVATION_CALIBRATION_SUSPENDED.reset(token)


def _module_fp8_input_scale(module: nn.Module, inputs: torch.Tensor) -> torch.Tensor | None:
    """FL/distributed/linear.py:104-128: None -> dynamic; during calibration the
    observed per-tensor scale (running max kept in ``_fp8_activation_scale``);
    afterwards the frozen scale times the margin, or the prefix-shared scale."""
    scale = getattr(module, "_fp8_activation_scale", None)
    if scale is None:
        return None
    suspended = _FP8_ACTIVATION_CALIBRATION_SUSPENDED.get()
    remaining = int(getattr(module, "_fp8_activation_calibration_remaining", 0))
    if remaining > 0 or suspended:
        observed = torch.clamp(inputs.detach().abs().amax().to(torch.float32) / 448.0, min=1.0e-12)
        if remaining > 0 and not suspended:
            torch.maximum(scale, observed, out=scale)
            module._fp8_activation_calibration_remaining = remaining - 1
        return observed
    margin = float(getattr(module, "_fp8_activation_scale_margin", 1.0))
    if _FP8_ACTIVATION_SCALE_POLICY.get() == "prefix_shared":
        prefix = getattr(module, "_fp8_prefix_activation_scale", None)
        if prefix is not None:
            return prefix * margin
    return scale * margin


__all__ = [
    "_cross_rank",
    "_linear",
    "_module_fp8_input_scale",
    "_module_linear",
    "suspend_fp8_activation_calibration",
    "use_fp8_activation_scale_policy",
]
