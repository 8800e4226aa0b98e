"""The reference's quantized-linear arithmetic as host torch code (TEST
INFRASTRUCTURE ONLY: used by tests/ as a second, library-evaluated statement
of the reference formulas and by bench.py's cpu_baseline leg).

Each function evaluates the reference's own torch expression, on CPU or GPU
tensors.  One operation needs care: the reference runs on the GPU, where
PyTorch's kernel for a tensor divided by a Python scalar (``amax / 127.0``,
``amax / FP8_MAX``) multiplies by the binary32 reciprocal of the scalar, while
on the CPU torch divides.  ``scalar_div`` evaluates that operation the device's
way on either; a GPU test checks that it equals ``t / c`` on the device over
every bf16 value.

* ``quantize_weight_int8``   H3/inference/w8a8.py:57-63
* ``quantize_rows_e4m3``     the same expression with 127 -> 448 and the
                             e4m3fn cast (per-token / per-channel FP8)
* ``quantize_tensor_e4m3``   FL/inference/fused_kernels.py:771-796 (eager)
* ``quantize_fp8_e4m3_per_head``  FL/inference/fused_kernels.py:823-834 (eager)
* ``quantize_act_int8_vllm`` vLLM's dynamic per-token int8 (H3/inference/w8a8.py:178)
* ``int8_linear``            torch._int_mm then s_a * (s_w * float(acc))
* ``fp8_linear``             dequant-then-matmul F.linear(q_a.float()*s_a,
                             q_w.float()*s_w, bias) -> bf16 (the CPU baseline)
* ``lora_update``            H3/inference/lora_checkpoint.py:196-205
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

FP8_MAX = 448.0


def scalar_div(t: torch.Tensor, c: float) -> torch.Tensor:
    """``t / c`` for a binary32 tensor as the GPU evaluates it: t * RN(1/c)."""
    if t.is_cuda:
        return t / c
    return t * (torch.tensor(1.0, dtype=torch.float32) / c)


def quantize_weight_int8(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    scale = torch.clamp(scalar_div(weight.abs().amax(dim=1, keepdim=True).float(), 127.0), min=1.0e-12)
    quantized = torch.clamp(torch.round(weight / scale), -127, 127).to(torch.int8)
    return quantized.contiguous(), scale.contiguous()


def quantize_rows_e4m3(value: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    scale = torch.clamp(scalar_div(value.abs().amax(dim=1, keepdim=True).float(), FP8_MAX), min=1.0e-12)
    quantized = torch.clamp(value / scale, -FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return quantized.contiguous(), scale.contiguous()


def quantize_tensor_e4m3(value: torch.Tensor, scale: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    # value / scale with a 0-dim fp32 scale computes in bf16: torch on the CPU
    # divides by the fp32 scale, torch on the GPU by the scale cast to bf16.
    if scale is None:
        scale = torch.clamp(scalar_div(value.detach().abs().amax().to(torch.float32), FP8_MAX), min=1.0e-12)
    return torch.clamp(value / scale, -FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn), scale


def quantize_fp8_e4m3_per_head(value: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    scale = torch.clamp(scalar_div(value.float().abs().amax(dim=(1, 3)), FP8_MAX), min=1.0e-12)
    quantized = torch.clamp(value / scale[:, None, :, None], -FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return quantized, scale


def quantize_act_int8_vllm(value: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """vLLM 0.11.1's published dynamic per-token int8 form (called at
    H3/inference/w8a8.py:178): s = amax / 127, q = sat8(rint(x * (127 / amax))),
    a zero row giving zero codes (TEST INFRASTRUCTURE: the CPU baseline's act-quant)."""
    amax = value.abs().amax(dim=1, keepdim=True).float()
    inv = torch.where(amax > 0, 127.0 / amax, torch.zeros_like(amax))
    quantized = torch.clamp(torch.round(value.float() * inv), -128, 127).to(torch.int8)
    return quantized.contiguous(), (amax / 127.0).contiguous()


def int8_linear(q_a: torch.Tensor, s_a: torch.Tensor, q_w: torch.Tensor, s_w: torch.Tensor) -> torch.Tensor:
    acc = torch._int_mm(q_a, q_w.t())
    return (s_a.view(-1, 1) * (s_w.view(1, -1) * acc.float())).to(torch.bfloat16)


def fp8_linear(q_a: torch.Tensor, s_a: torch.Tensor, q_w: torch.Tensor, s_w: torch.Tensor,
               bias: torch.Tensor | None = None) -> torch.Tensor:
    a = q_a.float() * s_a.view(-1, 1)
    w = q_w.float() * s_w.view(-1, 1)
    return F.linear(a, w, None if bias is None else bias.float()).to(torch.bfloat16)


def lora_update(inputs: torch.Tensor, output: torch.Tensor, lora_a: torch.Tensor, lora_b: torch.Tensor,
                scale: float) -> torch.Tensor:
    compute_dtype = output.dtype
    update = F.linear(F.linear(inputs.to(compute_dtype), lora_a), lora_b)
    return output + update * scale


def w8a8_fp8_linear_step(x: torch.Tensor, q_w: torch.Tensor, s_w: torch.Tensor,
                         bias: torch.Tensor | None) -> torch.Tensor:
    """One host step of the FP8 W8A8 linear: per-token act quant, then the
    dequant-then-matmul GEMM with bias (the CPU baseline of bench.py)."""
    q_a, s_a = quantize_rows_e4m3(x)
    return fp8_linear(q_a, s_a, q_w, s_w, bias)
