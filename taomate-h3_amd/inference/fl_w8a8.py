"""Int8 W8A8 for the FL2VA package's interior projections on MI355X.

Drop-in for ``digitalhuman_h3.inference.w8a8`` (FL/inference/w8a8.py:1-480),
the FL2VA twin of ``taomate_h3.inference.w8a8``.  Its functions take the
``torch`` module as their first argument and its receipts carry more keys;
the arithmetic is the same int8 W8A8 path as the H3 mirror
(``taomate_h3_amd.inference.w8a8``), on the gfx950 library:

* per-token activation codes: ``h3q_quant_rows`` (INT8, RCP_MUL), vLLM's
  ``dynamic_scaled_int8_quant`` semantics;
* per-output-channel weight codes: ``h3q_quant_rows`` / ``h3q_quant_rows_tiled``
  (INT8, DIV), the expression of FL/inference/w8a8.py:242-257;
* the GEMM: ``h3q_scaled_mm`` with ``s_a * (s_w * float(acc))`` -> bf16.

Beyond the H3 mirror this module adds FL's post-load conversion
(``quantize_h3_interior_qkv_fc1_linears_cutlass_w8a8_``, FL/inference/w8a8.py:340-466):
a BF16 projection that was not stream-loaded is quantized after loading,
and the whole selected set is validated before any parameter is replaced.
"""

from __future__ import annotations

from typing import Any

from .. import ops
from . import w8a8 as _h3

INTERIOR_FC1_QKV_CUTLASS_W8A8_POLICY = "interior_fc1_qkv_v1"
H3_CUTLASS_W8A8_POLICIES = (INTERIOR_FC1_QKV_CUTLASS_W8A8_POLICY,)
_STREAM_LOAD_TEMPORARY_BYTES = 8 * 1024 * 1024
_PROJECTION_SUFFIXES = (".attn.qkv_proj", ".mlp.fc1", ".mlp.fc2")
_QUANTIZED_SUFFIXES = (".attn.qkv_proj", ".mlp.fc1")

require_vllm_cutlass_w8a8 = _h3.require_vllm_cutlass_w8a8


class CutlassW8A8Workspace(_h3.CutlassW8A8Workspace):
    """Grow-only per-stream activation and output buffers (FL/inference/w8a8.py:13-116).

    The FL constructor takes the ``torch`` module; buffers, stream keys and
    the aliasing of same-width outputs are those of the H3 workspace."""

    def __init__(self, torch: Any) -> None:
        del torch
        super().__init__()


def resolve_h3_cutlass_w8a8_policy(linear_names: list[str], *, policy: str) -> dict[str, Any]:
    """FL's selection of the interior QKV/FC1 projections (FL/inference/w8a8.py:135-170).

    Unlike the H3 resolver it accepts any name ending in a projection suffix,
    reports the policy, and lists the boundary blocks as the first two and
    last three indices in that order."""
    if policy not in H3_CUTLASS_W8A8_POLICIES:
        raise ValueError("unsupported H3 CUTLASS W8A8 policy")
    projections = [name for name in linear_names if name.endswith(_PROJECTION_SUFFIXES)]
    if not projections:
        raise ValueError("H3 CUTLASS W8A8 policy requires projection candidates")
    indices = sorted({int(name.split(".", 2)[1]) for name in projections})
    boundary = [*indices[:2], *indices[-3:]]
    quantized = [name for name in projections
                 if name.endswith(_QUANTIZED_SUFFIXES) and int(name.split(".", 2)[1]) not in boundary]
    chosen = set(quantized)
    return {
        "policy": policy,
        "quantized_linear_names": quantized,
        "bf16_protected_linear_names": [name for name in projections if name not in chosen],
        "bf16_boundary_block_indices": boundary,
    }


def cutlass_w8a8_linear(torch: Any, inputs: Any, weight: Any, weight_scale: Any, *, bias: Any | None,
                        workspace: CutlassW8A8Workspace | None = None, weight_t: Any | None = None,
                        weight_scale_t: Any | None = None) -> Any:
    """Dynamic per-token int8 activations x per-channel int8 weights -> bf16
    (FL/inference/w8a8.py:173-207)."""
    del torch
    if bias is not None:
        raise RuntimeError("H3 CUTLASS W8A8 currently supports bias-free linears")
    return _h3.cutlass_w8a8_linear(inputs, weight, weight_scale, bias=None, workspace=workspace,
                                   weight_t=weight_t, weight_scale_t=weight_scale_t)


def enable_h3_cutlass_w8a8_workspace_(torch: Any, transformer: Any) -> dict[str, Any]:
    """One shared workspace and the transposed views on every W8 block linear
    (FL/inference/w8a8.py:210-239)."""
    require_vllm_cutlass_w8a8()
    modules = [module for name, module in transformer.named_modules()
               if name.startswith("blocks.") and getattr(module, "_cutlass_w8a8_weight_scale", None) is not None]
    if not modules:
        raise RuntimeError("CUTLASS W8A8 workspace requires quantized H3 linears")
    workspace = CutlassW8A8Workspace(torch)
    for module in modules:
        module._cutlass_w8a8_workspace = workspace
        module._cutlass_w8a8_weight_t = module.weight.t()
        module._cutlass_w8a8_weight_scale_t = module._cutlass_w8a8_weight_scale.t()
    return {
        "schema": "digitalhuman_h3.inference.cutlass_w8a8_workspace.v1",
        "linear_count": len(modules),
        "workspace_count_per_rank": 1,
        "allocation_policy": "grow_only_per_cuda_stream_and_shape",
        "activation_quantization": "unchanged_dynamic_per_token_symmetric",
        "weight_quantization": "unchanged_static_per_output_channel_symmetric",
        "arithmetic_order_changed": False,
    }


def _quantize_cutlass_w8a8_weight(torch: Any, weight: Any) -> tuple[Any, Any]:
    """Per-output-channel int8 codes and fp32 [N, 1] scales of a bf16 weight
    (FL/inference/w8a8.py:242-257), row-major."""
    if weight.dtype != torch.bfloat16:
        weight = weight.to(torch.bfloat16)
    return ops.quant_rows(weight.contiguous(), ops.FMT_INT8, ops.ROUND_DIV)


def _new_w8_parameter(torch: Any, weight: Any) -> tuple[Any, Any]:
    """Int8 codes of a bf16 device weight in the layout the GEMMs read best
    (tiled when the shape allows), with its scales."""
    rows, cols = int(weight.shape[0]), int(weight.shape[1])
    source = weight.detach()
    if source.dtype != torch.bfloat16:
        source = source.to(torch.bfloat16)
    source = source.contiguous()
    if ops.can_tile(rows, cols):
        codes, scale = ops.quant_rows_tiled(source, ops.FMT_INT8, ops.ROUND_DIV)
        parameter = torch.nn.Parameter(codes, requires_grad=False)
        ops.mark_tiled(parameter)
        return parameter, scale
    codes, scale = ops.quant_rows(source, ops.FMT_INT8, ops.ROUND_DIV)
    return torch.nn.Parameter(codes, requires_grad=False), scale


def prepare_cutlass_w8a8_stream_load_slot_(torch: Any, module: Any, *, name: str) -> None:
    """Give one projection its final W8 storage before loading (FL/inference/w8a8.py:260-293).

    A BF16 weight is replaced by an int8 parameter; an int8 weight allocated
    at construction (frozen) is kept."""
    weight = module.weight
    if weight.dtype not in (torch.bfloat16, torch.int8):
        raise TypeError(f"{name} expected an uninitialized BF16 or INT8 weight")
    if getattr(module, "bias", None) is not None:
        raise RuntimeError(f"{name} expected a bias-free H3 projection")
    if getattr(module, "_cutlass_w8a8_weight_scale", None) is not None:
        raise RuntimeError(f"{name} already owns CUTLASS W8A8 storage")
    rows, cols = int(weight.shape[0]), int(weight.shape[1])
    if weight.dtype == torch.bfloat16:
        module.weight = torch.nn.Parameter(torch.empty((rows, cols), dtype=torch.int8, device=weight.device),
                                           requires_grad=False)
    elif weight.requires_grad:
        raise RuntimeError(f"{name} preallocated INT8 weight requires gradients")
    if ops.can_tile(rows, cols):
        ops.mark_module_weight_tiled(module)
    module.register_buffer("_cutlass_w8a8_weight_scale",
                           torch.empty((rows, 1), dtype=torch.float32, device=weight.device), persistent=False)
    module._cutlass_w8a8_stream_load_pending = True
    module._cutlass_w8a8_stream_loaded = False
    module._cutlass_w8a8_source_weight_bytes = rows * cols * 2


def load_cutlass_w8a8_stream_weight_(torch: Any, module: Any, source_weight: Any, *, name: str,
                                     maximum_temporary_bytes: int = _STREAM_LOAD_TEMPORARY_BYTES) -> None:
    """Quantize a BF16 source tensor into a prepared W8 slot in bounded row
    chunks (FL/inference/w8a8.py:296-337); per-row scales make the chunked
    result equal to whole-matrix quantization."""
    if getattr(module, "_cutlass_w8a8_stream_load_pending", None) is not True:
        raise RuntimeError(f"{name} has no pending CUTLASS W8A8 stream load")
    if module.weight.dtype != torch.int8 or source_weight.dtype != torch.bfloat16:
        raise TypeError(f"{name} streamed CUTLASS W8A8 dtype differs")
    if tuple(module.weight.shape) != tuple(source_weight.shape):
        raise ValueError(f"{name} streamed CUTLASS W8A8 shape differs")
    if source_weight.ndim != 2:
        raise ValueError(f"{name} streamed CUTLASS W8A8 weight must be 2D")
    if maximum_temporary_bytes <= 0:
        raise ValueError("maximum_temporary_bytes must be positive")
    # The streamed writer keeps two device staging chunks of half the budget
    # each, so the device temporaries stay within the same bound.
    _h3.stream_quantize_rows_(module, int(source_weight.shape[0]), int(source_weight.shape[1]),
                              lambda start, stop: source_weight[start:stop], name=name,
                              maximum_temporary_bytes=int(maximum_temporary_bytes))


def _projection_modules(torch: Any, transformer: Any) -> list[tuple[str, Any]]:
    """(name, frozen base) for each ``blocks.*`` QKV/FC1/FC2 projection; a LoRA
    wrapper contributes its ``base`` so adapter switching keeps working."""
    found = []
    for name, module in transformer.named_modules():
        if not name.startswith("blocks.") or not name.endswith(_PROJECTION_SUFFIXES):
            continue
        base = getattr(module, "base", module)
        weight = getattr(base, "weight", None)
        if isinstance(base, torch.nn.Module) and isinstance(weight, torch.Tensor) and weight.ndim == 2:
            found.append((name, base))
    return found


def quantize_h3_interior_qkv_fc1_linears_cutlass_w8a8_(torch: Any, transformer: Any, *,
                                                       policy: str) -> dict[str, Any]:
    """Quantize (or validate the streamed W8 storage of) the interior QKV/FC1
    base linears and return FL's receipt (FL/inference/w8a8.py:340-466).

    Every selected projection is checked before any is converted, so a bad
    entry leaves the transformer untouched."""
    require_vllm_cutlass_w8a8()
    candidates = _projection_modules(torch, transformer)
    selection = resolve_h3_cutlass_w8a8_policy([name for name, _ in candidates], policy=policy)
    wanted = set(selection["quantized_linear_names"])
    selected = [(name, module) for name, module in candidates if name in wanted]
    if not selected:
        raise RuntimeError("H3 CUTLASS W8A8 policy selected no linears")

    streamed = set()
    for name, module in selected:
        if getattr(module, "_cutlass_w8a8_weight_scale", None) is not None:
            complete = (module.weight.dtype == torch.int8
                        and getattr(module, "_cutlass_w8a8_stream_load_pending", None) is False
                        and getattr(module, "_cutlass_w8a8_stream_loaded", None) is True)
            if not complete:
                raise RuntimeError(f"{name} has incomplete CUTLASS W8A8 storage")
            streamed.add(name)
        elif module.weight.dtype != torch.bfloat16:
            raise TypeError(f"{name} expected BF16 weight before W8A8 conversion")
        if getattr(module, "bias", None) is not None:
            raise RuntimeError(f"{name} expected a bias-free H3 projection")

    def source_bytes_of(module: Any) -> int:
        return int(getattr(module, "_cutlass_w8a8_source_weight_bytes",
                           module.weight.numel() * module.weight.element_size()))

    eligible = sum(source_bytes_of(module) for _, module in candidates)
    source_bytes = quantized_bytes = 0
    converted = []
    for name, module in selected:
        if name not in streamed:
            source_bytes += int(module.weight.numel() * module.weight.element_size())
            parameter, scale = _new_w8_parameter(torch, module.weight)
            module.weight = parameter
            if ops.is_tiled(parameter):
                ops.mark_module_weight_tiled(module)
            module.register_buffer("_cutlass_w8a8_weight_scale", scale, persistent=False)
        else:
            source_bytes += int(module._cutlass_w8a8_source_weight_bytes)
        quantized_bytes += int(module.weight.numel() * module.weight.element_size())
        converted.append(name)
    return {
        "schema": "digitalhuman_h3.inference.cutlass_w8a8.v1",
        "format": "int8_w8a8",
        "scope": "frozen_main_dit_base_weights_only",
        "policy": policy,
        "projection_set": "interior_qkv_and_fc1",
        "quantized_projection_suffixes": ["attn.qkv_proj", "mlp.fc1"],
        "activation_scale": "dynamic_per_token_symmetric",
        "weight_scale": "static_per_output_channel_symmetric",
        "kernel": "vllm_cutlass_scaled_mm",
        "eligible_linear_count": len(candidates),
        "linear_count": len(converted),
        "stream_load_linear_count": len(streamed),
        "bf16_protected_linear_count": len(selection["bf16_protected_linear_names"]),
        "quantized_linear_names": converted,
        "bf16_protected_linear_names": selection["bf16_protected_linear_names"],
        "bf16_boundary_block_indices": selection["bf16_boundary_block_indices"],
        "source_weight_bytes": source_bytes,
        "quantized_weight_bytes": quantized_bytes,
        "eligible_source_weight_bytes": eligible,
        "eligible_weight_fraction": source_bytes / eligible,
        "bf16_projection_suffixes": ["attn.out_proj", "mlp.fc2"],
        "lora_branch": {"storage": "fp32_online_unmodified", "compute": "bf16"},
        "base_teacher_adapter_bypass": "lora_only",
        "base_teacher_base_precision": "int8_w8a8",
        "runtime_state": "transient_not_checkpoint_reconstructible",
    }


__all__ = [
    "CutlassW8A8Workspace",
    "H3_CUTLASS_W8A8_POLICIES",
    "INTERIOR_FC1_QKV_CUTLASS_W8A8_POLICY",
    "cutlass_w8a8_linear",
    "enable_h3_cutlass_w8a8_workspace_",
    "load_cutlass_w8a8_stream_weight_",
    "prepare_cutlass_w8a8_stream_load_slot_",
    "quantize_h3_interior_qkv_fc1_linears_cutlass_w8a8_",
    "require_vllm_cutlass_w8a8",
    "resolve_h3_cutlass_w8a8_policy",
]
