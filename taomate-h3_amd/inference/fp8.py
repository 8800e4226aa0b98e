"""FP8 linears of the H3 DiT on gfx950.

Drop-in for FL/inference/fp8.py (policies, per-tensor dynamic/calibrated FP8
block linears, FP8DynamicLinear, cross-stage scale synchronisation), with the
same ``torch``-first signatures, module attributes and receipts.  Weight
quantization runs on the device through ``h3q_quant_tensor_e4m3`` and is
bit-identical to the reference expression (FL/inference/fp8.py:259-263).

``quantize_h3_block_linears_fp8_w8a8_`` adds the per-token x per-channel FP8
format (e4m3fn weights with one scale per output channel, dynamic per-token
activations) that has no counterpart in the reference; it marks a linear
with ``_fp8_w8a8_weight_scale [N, 1]`` and is dispatched by
``distributed.linear._module_linear``.
"""

from __future__ import annotations

from typing import Any

from .. import ops

QUALITY_FIRST_RESIDUAL_FP8_POLICY = "quality_first_residual_v1"
INTERIOR_FC1_ONLY_FP8_POLICY = "interior_fc1_only_v1"
INTERIOR_FC1_MID18_QKV_FP8_POLICY = "interior_fc1_mid18_qkv_v1"
H3_DYNAMIC_FP8_POLICIES = (
    QUALITY_FIRST_RESIDUAL_FP8_POLICY,
    INTERIOR_FC1_ONLY_FP8_POLICY,
    INTERIOR_FC1_MID18_QKV_FP8_POLICY,
)
H3_CALIBRATED_ONLY_FP8_POLICIES = (INTERIOR_FC1_ONLY_FP8_POLICY, INTERIOR_FC1_MID18_QKV_FP8_POLICY)
_INTERIOR_QKV_BLOCK_RANGES = {INTERIOR_FC1_MID18_QKV_FP8_POLICY: (16, 33)}


def _block(name: str) -> int:
    return int(name.split(".", 2)[1])


def resolve_h3_dynamic_fp8_policy(linear_names: list[str], *, policy: str | None) -> dict[str, Any]:
    """Select FP8 linears by policy (FL/inference/fp8.py:23-93).

    ``None`` quantizes every eligible name; the named policies keep the first
    two and last three blocks BF16, quantize the SwiGLU input projection of
    every other block, and quantize QKV in all of them (quality-first), in
    none (fc1-only) or in blocks 16..33 (mid18)."""
    if policy is not None and policy not in H3_DYNAMIC_FP8_POLICIES:
        raise ValueError("unsupported H3 dynamic FP8 policy")
    if not linear_names:
        raise ValueError("H3 dynamic FP8 policy requires eligible linear names")
    if policy is None:
        return {"quantized_linear_names": list(linear_names), "bf16_protected_linear_names": [],
                "bf16_boundary_block_indices": []}
    blocks = sorted({_block(n) for n in linear_names})
    boundary = tuple((*blocks[:2], *blocks[-3:]))

    def chosen(name: str) -> bool:
        b = _block(name)
        if b in boundary:
            return False
        if name.endswith(".mlp.fc1"):
            return True
        if not name.endswith(".attn.qkv_proj"):
            return False
        if policy == QUALITY_FIRST_RESIDUAL_FP8_POLICY:
            return True
        rng = _INTERIOR_QKV_BLOCK_RANGES.get(policy)
        return rng is not None and rng[0] <= b <= rng[1]

    quantized = [n for n in linear_names if chosen(n)]
    qset = set(quantized)
    qkv_q = sorted({_block(n) for n in quantized if n.endswith(".attn.qkv_proj")})
    qkv_all = {_block(n) for n in linear_names if n.endswith(".attn.qkv_proj")}
    return {
        "quantized_linear_names": quantized,
        "bf16_protected_linear_names": [n for n in linear_names if n not in qset],
        "bf16_boundary_block_indices": list(boundary),
        "quantized_qkv_block_indices": qkv_q,
        "bf16_qkv_block_indices": sorted(qkv_all - set(qkv_q)),
    }


# Receipt vocabulary of FL/inference/fp8.py:288-372: which projections a
# policy covers, the reason it gives, and the components FP8 never touches.
_PROJECTION_SETS = {
    INTERIOR_FC1_ONLY_FP8_POLICY: "mlp_input_interior_blocks",
    INTERIOR_FC1_MID18_QKV_FP8_POLICY: "mlp_input_interior_and_mid18_qkv_blocks",
    QUALITY_FIRST_RESIDUAL_FP8_POLICY: "qkv_and_mlp_input_interior_blocks",
}
_EXCLUDED_COMPONENTS = ("lora_adapter_tensors", "patch_projections", "timestep_projections",
                        "final_output_projections", "token_refiner", "condition_and_adaln")
_BOUNDARY_REASON = "both representation boundaries"


def _projection_set(policy: str | None, mlp_only: bool) -> str:
    return "mlp_only" if mlp_only else _PROJECTION_SETS.get(policy, "attention_and_mlp")


def _policy_rules(policy: str | None, selection: dict[str, Any]) -> dict[str, Any] | None:
    """What a named policy quantizes and protects, for the receipt; None
    without a named policy."""
    if policy not in H3_DYNAMIC_FP8_POLICIES:
        return None
    fc1_only = policy == INTERIOR_FC1_ONLY_FP8_POLICY
    if fc1_only:
        reason = ("protect attention, residual-write projections, and " + _BOUNDARY_REASON
                  + " (first two and last three blocks)")
    elif policy in _INTERIOR_QKV_BLOCK_RANGES:
        lo, hi = _INTERIOR_QKV_BLOCK_RANGES[policy]
        reason = (f"protect QKV outside blocks {lo} through {hi}, all residual-write projections, and "
                  + _BOUNDARY_REASON)
    else:
        reason = "protect residual-write projections and " + _BOUNDARY_REASON + " (first two and last three blocks)"
    quantized = ["mlp.fc1"] if fc1_only else ["attn.qkv_proj", "mlp.fc1"]
    return {
        "quantized_projection_suffixes": quantized,
        "bf16_projection_suffixes": [s for s in ("attn.qkv_proj", "attn.out_proj", "mlp.fc2") if s not in quantized],
        "bf16_boundary_block_indices": selection["bf16_boundary_block_indices"],
        "quantized_qkv_block_indices": selection["quantized_qkv_block_indices"],
        "bf16_qkv_block_indices": selection["bf16_qkv_block_indices"],
        "reason": reason,
    }


def quantize_weight_fp8_tensor(weight: Any) -> tuple[Any, Any]:
    """Per-tensor e4m3fn weight codes and 0-dim fp32 scale (FL/inference/fp8.py:259-263,
    :107-113): the eager expression as torch evaluates it on the GPU, so the
    quotient's divisor is the scale rounded to bf16."""
    return ops.quant_tensor_e4m3(weight.detach().contiguous(), bf16_divisor=True)


def quantize_weight_fp8_rows(weight: Any) -> tuple[Any, Any]:
    """Per-output-channel e4m3fn weight codes [N, K] and fp32 scales [N, 1]."""
    return ops.quant_rows(weight.detach().contiguous(), ops.FMT_E4M3FN, ops.ROUND_DIV)


class FP8DynamicLinear:
    """Inference-only FP8 replacement for an aligned ``torch.nn.Linear``
    (FL/inference/fp8.py:96-146).

    As in the reference, everything is quantized in its own dtype: the
    source weight (bf16, fp16 or fp32; the video VAE that uses this module
    loads fp32) with the eager expression ``clamp(w / s)`` in that dtype, the
    activations per call by ``quantize_fp8_e4m3_dynamic`` in theirs (fp16
    under the VAE's autocast).  The bias is kept as fp16 and the GEMM
    rounds ``s_x * (s_w * acc) + bias`` once to fp16, as
    ``torch._scaled_mm(..., bias=fp16, out_dtype=torch.float16)``."""

    @staticmethod
    def from_linear(torch: Any, source: Any) -> Any:
        class _FP8DynamicLinear(torch.nn.Module):
            def __init__(self) -> None:
                super().__init__()
                quantized, scale = ops.quant_tensor_e4m3(source.weight.detach().contiguous(), eager=True)
                self.weight = torch.nn.Parameter(quantized, requires_grad=False)
                self.register_buffer("weight_scale", scale, persistent=True)
                self.bias = (torch.nn.Parameter(source.bias.detach().to(torch.float16), requires_grad=False)
                             if source.bias is not None else None)
                self.in_features = int(source.in_features)
                self.out_features = int(source.out_features)

            def forward(self, value: Any) -> Any:
                from .fused_kernels import quantize_fp8_e4m3_dynamic

                shape = (*value.shape[:-1], self.out_features)
                flattened = value.reshape(-1, self.in_features)
                quantized, input_scale = quantize_fp8_e4m3_dynamic(flattened)
                output = ops.scaled_mm(quantized, self.weight, input_scale.reshape(1), self.weight_scale.reshape(1),
                                       bias=self.bias, out_dtype=torch.float16)
                return output.reshape(shape)

        return _FP8DynamicLinear()


def quantize_aligned_linears_dynamic_fp8_(torch: Any, module: Any) -> dict[str, Any]:
    """Replace 16-aligned Linear children with dynamic FP8 modules (FL/inference/fp8.py:149-183)."""
    names: list[str] = []

    def visit(parent: Any, prefix: str) -> None:
        for child_name, child in list(parent.named_children()):
            qualified = f"{prefix}.{child_name}" if prefix else child_name
            if (isinstance(child, torch.nn.Linear) and int(child.in_features) % 16 == 0
                    and int(child.out_features) % 16 == 0):
                setattr(parent, child_name, FP8DynamicLinear.from_linear(torch, child))
                names.append(qualified)
            else:
                visit(child, qualified)

    visit(module, "")
    if not names:
        raise RuntimeError("no aligned Linear modules were selected for FP8")
    return {"schema": "digitalhuman_h3.inference.module_fp8_linear.v1", "format": "float8_e4m3fn",
            "activation_scale": "dynamic_per_tensor", "weight_scale": "static_per_tensor",
            "linear_count": len(names)}


def _is_parallel_linear(module: Any) -> bool:
    """A tensor-parallel linear of the reference (column, merged-column or
    row): a module with a 2-D weight and the ``input_size`` / ``output_size``
    those classes carry (FL/distributed/linear.py:131-181)."""
    weight = getattr(module, "weight", None)
    return getattr(weight, "ndim", 0) == 2 and hasattr(module, "input_size") and hasattr(module, "output_size")


def _block_candidates(transformer: Any, suffixes: tuple[str, ...]) -> list[tuple[str, Any]]:
    found = []
    for name, module in transformer.named_modules():
        if not name.startswith("blocks.") or not name.endswith(suffixes):
            continue
        base = getattr(module, "base", module)
        if _is_parallel_linear(base):
            found.append((name, base))
    return found


def _quantize_h3_block_linears_fp8_(torch: Any, transformer: Any, *, activation_calibration_forwards: int | None,
                                    activation_scale_margin: float, mlp_only: bool = False,
                                    policy: str | None = None) -> dict[str, Any]:
    """Quantize DiT block linears to per-tensor FP8 in place (FL/inference/fp8.py:186-374)."""
    if mlp_only and policy is not None:
        raise ValueError("H3 dynamic FP8 policy cannot be combined with MLP-only FP8")
    if activation_calibration_forwards is None and policy in H3_CALIBRATED_ONLY_FP8_POLICIES:
        raise ValueError(f"{policy} requires calibrated FP8 activation scales")
    suffixes = ((".mlp.fc1", ".mlp.fc2") if mlp_only
                else (".attn.qkv_proj", ".attn.out_proj", ".mlp.fc1", ".mlp.fc2"))
    candidates = _block_candidates(transformer, suffixes)
    if not candidates:
        raise RuntimeError("no H3 DiT block linears were selected for FP8")
    selection = resolve_h3_dynamic_fp8_policy([n for n, _ in candidates], policy=policy)
    wanted = set(selection["quantized_linear_names"])
    chosen = [(n, m) for n, m in candidates if n in wanted]
    if not chosen:
        raise RuntimeError("H3 dynamic FP8 policy selected no block linears")
    eligible = sum(int(m.weight.numel() * m.weight.element_size()) for _, m in candidates)
    names: list[str] = []
    source_bytes = quantized_bytes = 0
    for name, module in chosen:
        weight = module.weight.detach()
        if weight.dtype != torch.bfloat16:
            raise TypeError(f"{name} expected BF16 weight before FP8 conversion")
        quantized, scale = quantize_weight_fp8_tensor(weight)
        source_bytes += int(weight.numel() * weight.element_size())
        quantized_bytes += int(quantized.numel() * quantized.element_size())
        module.weight = torch.nn.Parameter(quantized, requires_grad=False)
        module.register_buffer("_fp8_weight_scale", scale, persistent=True)
        if activation_calibration_forwards is not None:
            module.register_buffer("_fp8_activation_scale",
                                   torch.zeros((), dtype=torch.float32, device=weight.device), persistent=False)
            module._fp8_activation_calibration_remaining = activation_calibration_forwards
            module._fp8_activation_scale_margin = activation_scale_margin
        names.append(name)
    protected = selection["bf16_protected_linear_names"]
    calibrated = activation_calibration_forwards is not None
    return {
        "schema": "digitalhuman_h3.inference.fp8.v3",
        "scope": "frozen_main_dit_base_weights_only",
        "excluded_components": list(_EXCLUDED_COMPONENTS),
        "format": "float8_e4m3fn",
        "activation_scale": "calibrated_static_per_tensor" if calibrated else "dynamic_per_tensor",
        "activation_calibration_forwards": activation_calibration_forwards,
        "activation_scale_margin": activation_scale_margin,
        "activation_calibration_scope": "student_av_forwards_only" if calibrated else None,
        "base_model_bypass_forwards": ("per_forward_scale_without_consuming_calibration" if calibrated else None),
        "weight_scale": "static_per_tensor",
        "projection_set": _projection_set(policy, mlp_only),
        "policy": policy or ("mlp_only_v1" if mlp_only else "all_main_blocks_v1"),
        "policy_rules": _policy_rules(policy, selection),
        "eligible_linear_count": len(candidates),
        "linear_count": len(names),
        "bf16_protected_linear_count": len(protected),
        "quantized_linear_names": names,
        "bf16_protected_linear_names": protected,
        "eligible_source_weight_bytes": eligible,
        "source_weight_bytes": source_bytes,
        "quantized_weight_bytes": quantized_bytes,
        "eligible_weight_fraction": source_bytes / eligible,
    }


def quantize_h3_block_linears_dynamic_fp8_(torch: Any, transformer: Any, *, policy: str | None = None) -> dict:
    return _quantize_h3_block_linears_fp8_(torch, transformer, activation_calibration_forwards=None,
                                           activation_scale_margin=1.0, policy=policy)


def quantize_h3_mlp_linears_dynamic_fp8_(torch: Any, transformer: Any) -> dict:
    """Quantize only MLP projections, leaving Q/K/V and attention output BF16."""
    return _quantize_h3_block_linears_fp8_(torch, transformer, activation_calibration_forwards=None,
                                           activation_scale_margin=1.0, mlp_only=True)


def quantize_h3_block_linears_calibrated_fp8_(torch: Any, transformer: Any, *, calibration_forwards: int = 5,
                                              scale_margin: float = 1.25, policy: str | None = None) -> dict:
    if calibration_forwards < 1:
        raise ValueError("FP8 calibration forwards must be positive")
    if scale_margin < 1.0:
        raise ValueError("FP8 activation scale margin must be at least one")
    return _quantize_h3_block_linears_fp8_(torch, transformer, activation_calibration_forwards=calibration_forwards,
                                           activation_scale_margin=scale_margin, policy=policy)


def synchronize_h3_block_fp8_activation_scales_(torch: Any, transformer: Any, *, group: Any) -> dict[str, Any]:
    """Publish one MAX-reduced clean-prefix scale per calibrated block linear
    (FL/inference/fp8.py:428-478).  ``group`` is a torch.distributed process
    group, or None when there is a single stage (the reduction is then the
    identity)."""
    selected = []
    for name, module in transformer.named_modules():
        scale = getattr(module, "_fp8_activation_scale", None)
        if not name.startswith("blocks.") or scale is None:
            continue
        if int(getattr(module, "_fp8_activation_calibration_remaining", 0)) != 0:
            raise RuntimeError("calibrated FP8 activation scales must be frozen before cross-stage synchronization")
        selected.append((module, scale))
    if not selected:
        raise RuntimeError("no calibrated H3 block-linear activation scales found")
    packed = torch.stack([s.detach().to(dtype=torch.float32) for _, s in selected])
    collectives = 0
    if group is not None:
        torch.distributed.all_reduce(packed, op=torch.distributed.ReduceOp.MAX, group=group)
        collectives = 1
    for index, (module, _) in enumerate(selected):
        prefix = getattr(module, "_fp8_prefix_activation_scale", None)
        if prefix is None:
            module.register_buffer("_fp8_prefix_activation_scale", packed[index].detach().clone(), persistent=False)
        else:
            prefix.copy_(packed[index])
    return {"enabled": True, "schema": "digitalhuman_h3.inference.fp8_stage_scale_sync.v2",
            "linear_count": len(selected), "collective_count": collectives, "reduction": "max",
            "group_scope": "corresponding_tp_lane_across_three_denoise_stages",
            "calibration_state": "frozen_before_sync", "target": "clean_prefix_only",
            "current_stage_scales_changed": False}


def quantize_h3_block_linears_fp8_w8a8_(torch: Any, transformer: Any, *, policy: str | None = None) -> dict:
    """Per-output-channel e4m3fn weights + dynamic per-token e4m3fn activations
    for the selected block linears (no counterpart in the reference; the
    format of the BASELINE.json FP8 W8A8 configurations).  Bias is kept (bf16) and
    fused into the GEMM epilogue.  Weights with N % 16 == 0 and K % 128 == 0
    are stored in the tiled layout (``ops.is_tiled(weight)``)."""
    candidates = _block_candidates(transformer, (".attn.qkv_proj", ".attn.out_proj", ".mlp.fc1", ".mlp.fc2"))
    if not candidates:
        raise RuntimeError("no H3 DiT block linears were selected for FP8 W8A8")
    selection = resolve_h3_dynamic_fp8_policy([n for n, _ in candidates], policy=policy)
    wanted = set(selection["quantized_linear_names"])
    names, source_bytes, quantized_bytes = [], 0, 0
    for name, module in candidates:
        if name not in wanted:
            continue
        weight = module.weight.detach()
        if weight.dtype != torch.bfloat16:
            raise TypeError(f"{name} expected BF16 weight before FP8 W8A8 conversion")
        tiled = ops.can_tile(int(weight.shape[0]), int(weight.shape[1]))
        if tiled:
            quantized, scale = ops.quant_rows_tiled(weight.contiguous(), ops.FMT_E4M3FN, ops.ROUND_DIV)
        else:
            quantized, scale = quantize_weight_fp8_rows(weight)
        source_bytes += int(weight.numel() * weight.element_size())
        quantized_bytes += int(quantized.numel() * quantized.element_size())
        module.weight = torch.nn.Parameter(quantized, requires_grad=False)
        if tiled:
            ops.mark_module_weight_tiled(module)
        module.register_buffer("_fp8_w8a8_weight_scale", scale, persistent=False)
        names.append(name)
    if not names:
        raise RuntimeError("H3 FP8 W8A8 policy selected no block linears")
    return {"format": "float8_e4m3fn_w8a8", "activation_scale": "dynamic_per_token",
            "weight_scale": "static_per_output_channel", "policy": policy or "all_main_blocks_v1",
            "linear_count": len(names), "quantized_linear_names": names,
            "bf16_protected_linear_names": selection["bf16_protected_linear_names"],
            "source_weight_bytes": source_bytes, "quantized_weight_bytes": quantized_bytes}


__all__ = [
    "FP8DynamicLinear",
    "H3_CALIBRATED_ONLY_FP8_POLICIES",
    "H3_DYNAMIC_FP8_POLICIES",
    "INTERIOR_FC1_MID18_QKV_FP8_POLICY",
    "INTERIOR_FC1_ONLY_FP8_POLICY",
    "QUALITY_FIRST_RESIDUAL_FP8_POLICY",
    "quantize_aligned_linears_dynamic_fp8_",
    "quantize_h3_block_linears_calibrated_fp8_",
    "quantize_h3_block_linears_dynamic_fp8_",
    "quantize_h3_block_linears_fp8_w8a8_",
    "quantize_h3_mlp_linears_dynamic_fp8_",
    "resolve_h3_dynamic_fp8_policy",
    "synchronize_h3_block_fp8_activation_scales_",
]
