"""Inference LoRA side branch on a quantized base linear.

Drop-in for the inference part of H3/inference/lora_checkpoint.py:172-205 and
:261-303 (wrapper, bf16 buffer materialisation, fused row reduction).  The
reference computes the base linear, then two bf16 ``F.linear`` calls and two
elementwise passes over the [M, N] output:

    output + F.linear(F.linear(x, A), B) * scale

When the base is a W8A8 linear (int8 or per-channel FP8) and the adapter
rank is at most 128, this wrapper instead computes t = bf16(x @ A^T) with
``h3q_lora_down`` and lets ``h3q_scaled_mm`` add ``scale * t @ B^T`` in the
GEMM epilogue before the single bf16 rounding of the output.  Other cases
(a BF16 base, rank above 128) keep the reference's two-GEMM formula.
Checkpoint loading (lora_checkpoint.py:61-150) stays the reference's:
``fuse_h3_lora_wrappers_`` swaps the wrappers its ``apply_h3_lora_checkpoint``
installed for this one.
"""

from __future__ import annotations

from collections.abc import Iterator
from contextlib import contextmanager
from typing import Any, Mapping

import torch
import torch.nn.functional as F

from .. import ops

FUSED_MAX_RANK = 128


class H3LoRACheckpointError(RuntimeError):
    """Raised for adapter shapes or targets the wrapper cannot serve."""


def _fusable_shape(base: Any, lora_a: torch.Tensor) -> bool:
    """A W8A8 base (int8 or per-channel FP8) and a rank the GEMM epilogue takes."""
    quantized = (getattr(base, "_cutlass_w8a8_weight_scale", None) is not None
                 or getattr(base, "_fp8_w8a8_weight_scale", None) is not None)
    rank = int(lora_a.shape[0])
    return quantized and 0 < rank <= FUSED_MAX_RANK and rank % 8 == 0 and lora_a.is_cuda


def _fusable(base: Any, lora_a: torch.Tensor, lora_b: torch.Tensor) -> bool:
    return (_fusable_shape(base, lora_a) and lora_a.dtype == torch.bfloat16
            and lora_b.dtype == torch.bfloat16)


def fused_quantized_lora_linear(base: Any, inputs: torch.Tensor, lora_a: torch.Tensor, lora_b: torch.Tensor,
                                scale: float) -> torch.Tensor:
    """base(x) + scale * (x @ A^T) @ B^T with one bf16 rounding, for a W8A8 base."""
    shape = (*inputs.shape[:-1], int(base.weight.shape[0]))
    ops.module_weight_tiled(base)  # re-marks the storage of a deep-copied tiled weight
    flat = inputs.reshape(-1, int(inputs.shape[-1]))
    if flat.dtype != torch.bfloat16:
        flat = flat.to(torch.bfloat16)
    flat = flat.contiguous()
    t = ops.lora_down(flat, lora_a.contiguous())
    bias = getattr(base, "bias", None)
    if getattr(base, "_cutlass_w8a8_weight_scale", None) is not None:
        if bias is not None:
            raise RuntimeError("H3 W8A8 supports bias-free linears only")
        workspace = getattr(base, "_cutlass_w8a8_workspace", None)
        if workspace is not None:
            _, s, out = workspace.buffers(flat, int(base.weight.shape[0]))
            q = workspace._codes_buffer(flat)
        else:
            q = s = out = None
        q, s, a_tiled = ops.quant_activations_for(flat, ops.FMT_INT8, ops.ROUND_RCP_MUL, base.weight, codes=q,
                                                  scales=s, lora=True)
        w_scale = base._cutlass_w8a8_weight_scale
    else:
        q, s, a_tiled = ops.quant_activations_for(flat, ops.FMT_E4M3FN, ops.ROUND_DIV, base.weight, lora=True)
        out = None
        w_scale = base._fp8_w8a8_weight_scale
    out = ops.scaled_mm(q, base.weight, s.reshape(-1), w_scale.reshape(-1), bias=bias, lora_t=t,
                        lora_b=lora_b.contiguous(), lora_scale=float(scale), out=out, a_tiled=a_tiled,
                        b_tiled=ops.module_weight_tiled(base), m=int(flat.shape[0]))
    return out.reshape(shape)


class H3InferenceParallelLinearLoRA(torch.nn.Module):
    """LoRA wrapper of a column- or row-parallel base linear
    (H3/inference/lora_checkpoint.py:172-205; FL/inference/lora_checkpoint.py:440-489).

    ``adapter_enabled`` (FL) switches the side branch off: the wrapper then
    returns the base output alone.  A row-parallel base split over several
    tensor-parallel ranks needs the cross-rank reduction of its partial
    output (with the LoRA partial added before it), which this single-GPU
    build does not perform: such a call raises instead of returning a
    partial sum."""

    def __init__(self, base: Any, *, kind: str, a: torch.Tensor, b: torch.Tensor, scale: float) -> None:
        super().__init__()
        if kind not in ("column", "row"):
            raise H3LoRACheckpointError(f"unknown LoRA target kind {kind}")
        self.base = base
        self.kind = kind
        self.scale = float(scale)
        self.adapter_enabled = True
        self.fused_row_reduce_enabled = False
        self._taomate_h3_inference_lora = True
        self.register_buffer("lora_a", a, persistent=False)
        self.register_buffer("lora_b", b, persistent=False)

    def forward(self, inputs: torch.Tensor) -> torch.Tensor:
        from .fused_kernels import as_dense

        if not self.adapter_enabled:
            return self.base(inputs)
        if self.kind == "row" and int(getattr(self.base, "tp_size", 1)) > 1:
            from ..distributed.linear import _cross_rank

            raise _cross_rank("reducing a row-parallel LoRA output")
        inputs = as_dense(inputs)  # the LoRA branch needs the bf16 rows
        if _fusable(self.base, self.lora_a, self.lora_b):
            return fused_quantized_lora_linear(self.base, inputs, self.lora_a, self.lora_b, self.scale)
        output = self.base(inputs)
        compute_dtype = output.dtype
        update = F.linear(F.linear(inputs.to(compute_dtype), self.lora_a.to(compute_dtype)),
                          self.lora_b.to(compute_dtype))
        if tuple(update.shape) != tuple(output.shape):
            raise H3LoRACheckpointError("H3 inference LoRA output shape differs")
        return output + update * self.scale


def materialize_h3_lora_bf16_buffers_(transformer: Any) -> Mapping[str, Any]:
    """Materialize the inference LoRA buffers once in bf16 (H3/inference/lora_checkpoint.py:261-284)."""
    adapters = [m for m in transformer.modules() if getattr(m, "_taomate_h3_inference_lora", False)]
    if not adapters:
        raise H3LoRACheckpointError("BF16 LoRA buffers require a loaded adapter")
    converted = 0
    for module in adapters:
        for name in ("lora_a", "lora_b"):
            value = getattr(module, name)
            if value.dtype != torch.bfloat16:
                converted += int(value.numel())
                setattr(module, name, value.to(dtype=torch.bfloat16))
    return {"target_count": len(adapters), "buffer_count": 2 * len(adapters), "converted_numel": converted,
            "dtype": "bfloat16"}


def enable_h3_fused_lora_row_reduce_(transformer: Any) -> Mapping[str, Any]:
    """Mark row-parallel adapters for the pre-reduction LoRA add (H3/inference/lora_checkpoint.py:287-303)."""
    rows = [m for m in transformer.modules()
            if getattr(m, "_taomate_h3_inference_lora", False) and getattr(m, "kind", None) == "row"]
    if not rows:
        raise H3LoRACheckpointError("fused row reduction requires a loaded adapter")
    for module in rows:
        module.fused_row_reduce_enabled = True
    return {"row_parallel_module_count": len(rows), "tp_all_reduce_calls_saved_per_forward": len(rows)}


def _adapters(transformer: Any) -> list[tuple[str, Any]]:
    return [(name, module) for name, module in transformer.named_modules()
            if getattr(module, "_taomate_h3_inference_lora", False)]


# The marker attributes the two reference packages set on their wrappers
# (H3/inference/lora_checkpoint.py:179, FL/inference/lora_checkpoint.py:448);
# their bf16-materialise, row-reduce, merge and base-model functions find the
# adapters by these names.
LORA_WRAPPER_MARKERS = ("_taomate_h3_inference_lora", "_digitalhuman_h3_inference_lora")


def _wrapper_markers(module: Any) -> tuple[str, ...]:
    return tuple(marker for marker in LORA_WRAPPER_MARKERS if getattr(module, marker, False) is True)


def fuse_h3_lora_wrappers_(transformer: Any) -> Mapping[str, Any]:
    """Swap the LoRA wrappers the reference installed for ``H3InferenceParallelLinearLoRA``.

    ``apply_h3_lora_checkpoint`` (H3/inference/lora_checkpoint.py:153-258;
    FL/inference/lora_checkpoint.py:417-568) builds its wrapper class inside
    the function and installs one instance per target with ``setattr``
    (H3 :238-246).  That class computes the base linear and then the two
    unfused ``F.linear`` calls and elementwise passes.  This function finds
    every module carrying either package's wrapper marker and replaces it, in
    its parent, with this package's wrapper holding the same ``base``,
    ``kind``, ``scale``, ``lora_a`` / ``lora_b`` buffers (the same tensors),
    ``fused_row_reduce_enabled``, ``adapter_enabled`` and markers, so the
    reference's later passes (``materialize_h3_lora_bf16_buffers_``,
    ``enable_h3_fused_lora_row_reduce_``, ``quantize_h3_interior_qkv_fc1_``'s
    ``getattr(module, "base", module)``) see what they expect.  On a W8A8
    base with a bf16 adapter of rank <= 128 the forward then adds the LoRA in
    the GEMM epilogue (checked when the forward runs, so the order against the
    bf16 materialisation and the W8A8 conversion does not matter).

    A row-parallel wrapper whose base spans several tensor-parallel ranks is
    left in place: its output needs the cross-rank reduction, which this
    package does not perform.  Every wrapper is validated before any is
    replaced; a wrapper that is already this package's is counted, not
    replaced.  Call it after ``apply_h3_lora_checkpoint`` (H3/runtime/direct.py:116,
    FL/runtime/direct.py:333) and before the acceleration profile runs."""
    found = [(name, module) for name, module in transformer.named_modules()
             if name and _wrapper_markers(module)]
    if not found:
        raise H3LoRACheckpointError("fusing LoRA wrappers requires a loaded inference LoRA adapter")
    plans, already, kept = [], 0, []
    for name, module in found:
        if isinstance(module, H3InferenceParallelLinearLoRA):
            already += 1
            continue
        for attr in ("base", "kind", "scale", "lora_a", "lora_b"):
            if not hasattr(module, attr):
                raise H3LoRACheckpointError(f"H3 inference LoRA wrapper lacks {attr}: {name}")
        kind = module.kind
        if kind not in ("column", "row"):
            raise H3LoRACheckpointError(f"unknown LoRA target kind {kind}: {name}")
        base, lora_a, lora_b = module.base, module.lora_a, module.lora_b
        weight = getattr(base, "weight", None)
        if weight is None or lora_a.ndim != 2 or lora_b.ndim != 2 or int(lora_a.shape[0]) != int(lora_b.shape[1]):
            raise H3LoRACheckpointError(f"H3 inference LoRA local shape differs: {name}")
        if int(lora_a.shape[1]) != int(weight.shape[1]) or int(lora_b.shape[0]) != int(weight.shape[0]):
            raise H3LoRACheckpointError(f"H3 inference LoRA local shape differs: {name}")
        if kind == "row" and int(getattr(base, "tp_size", 1)) > 1:
            kept.append(name)
            continue
        plans.append((name, module))
    fusable = 0
    for name, module in plans:
        parent = transformer
        parts = name.split(".")
        for part in parts[:-1]:
            parent = getattr(parent, part)
        if getattr(parent, parts[-1]) is not module:
            raise H3LoRACheckpointError(f"H3 inference LoRA target changed: {name}")
        replacement = H3InferenceParallelLinearLoRA(module.base, kind=module.kind, a=module.lora_a,
                                                    b=module.lora_b, scale=float(module.scale))
        replacement.fused_row_reduce_enabled = bool(getattr(module, "fused_row_reduce_enabled", False))
        replacement.adapter_enabled = bool(getattr(module, "adapter_enabled", True))
        for marker in _wrapper_markers(module):
            setattr(replacement, marker, True)
        replacement.train(module.training)
        setattr(parent, parts[-1], replacement)
        if _fusable_shape(replacement.base, replacement.lora_a):
            fusable += 1
    return {
        "schema": "taomate_h3_amd.inference.fused_lora_wrappers.v1",
        "target_count": len(found),
        "replaced_count": len(plans),
        "already_fused_wrapper_count": already,
        "kept_reference_wrapper_names": kept,
        # W8A8 bases whose adapter the epilogue takes once its buffers are bf16
        "fused_epilogue_ready_count": fusable,
        "fused_max_rank": FUSED_MAX_RANK,
    }


def merge_h3_lora_weights_(transformer: Any) -> Mapping[str, Any]:
    """Fold each loaded adapter into its frozen base weight (FL/inference/lora_checkpoint.py:642-706):
    W' = round_to_base_dtype(fp32(W) + scale * fp32(B) @ fp32(A)), once.  The
    adapter is then switched off and its buffers released.  Quantized (W8)
    bases cannot be merged (FL forbids the merge with W8A8,
    FL/inference/acceleration.py:103-104)."""
    adapters = _adapters(transformer)
    if not adapters:
        raise H3LoRACheckpointError("LoRA weight merge requires a loaded inference LoRA adapter")
    merged_numel = released = 0
    for name, module in adapters:
        if not bool(module.adapter_enabled):
            raise H3LoRACheckpointError(f"H3 inference LoRA target is already disabled: {name}")
        weight = module.base.weight.detach()
        if weight.dtype not in (torch.bfloat16, torch.float16, torch.float32):
            raise H3LoRACheckpointError(f"H3 inference LoRA base weight cannot be merged: {name}")
        if int(module.lora_a.shape[1]) != int(weight.shape[1]) or int(module.lora_b.shape[0]) != int(weight.shape[0]):
            raise H3LoRACheckpointError(f"H3 inference LoRA local merge shape differs: {name}")
        delta = module.lora_b.float() @ module.lora_a.float()
        merged = (weight.float() + delta * float(module.scale)).to(weight.dtype)
        module.base.weight = torch.nn.Parameter(merged, requires_grad=False)
        merged_numel += int(merged.numel())
        released += int(module.lora_a.numel() + module.lora_b.numel())
        module.adapter_enabled = False
        module._taomate_h3_lora_merged = True
        del module.lora_a
        del module.lora_b
    return {
        "schema": "digitalhuman_h3.inference.lora_weight_merge.v1",
        "arithmetic": "fp32_delta_and_accumulate_then_round_to_base_dtype",
        "target_count": len(adapters),
        "merged_weight_numel": merged_numel,
        "released_adapter_numel": released,
        "online_lora_gemms_removed_per_forward": 2 * len(adapters),
        "reversible": False,
    }


@contextmanager
def h3_base_model_inference(transformer: Any) -> Iterator[None]:
    """Run the base model with every adapter switched off, without consuming
    FP8 activation-calibration samples (FL/inference/lora_checkpoint.py:709-739)."""
    from ..distributed.linear import suspend_fp8_activation_calibration

    modules = [module for _, module in _adapters(transformer)]
    if not modules:
        raise H3LoRACheckpointError("Base audio teacher requires an inference LoRA checkpoint")
    if any(getattr(module, "_taomate_h3_lora_merged", False) for module in modules):
        raise H3LoRACheckpointError("Base audio teacher cannot bypass an already merged LoRA weight")
    previous = [bool(module.adapter_enabled) for module in modules]
    for module in modules:
        module.adapter_enabled = False
    try:
        with suspend_fp8_activation_calibration():
            yield
    finally:
        for module, enabled in zip(modules, previous):
            module.adapter_enabled = enabled


__all__ = [
    "h3_base_model_inference",
    "merge_h3_lora_weights_",
    "FUSED_MAX_RANK",
    "H3InferenceParallelLinearLoRA",
    "H3LoRACheckpointError",
    "enable_h3_fused_lora_row_reduce_",
    "fused_quantized_lora_linear",
    "fuse_h3_lora_wrappers_",
    "LORA_WRAPPER_MARKERS",
    "materialize_h3_lora_bf16_buffers_",
]
