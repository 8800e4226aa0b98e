"""Minimal tensor-parallel linear layers for the tests (test scaffolding only).

The product package replaces only the quantized-linear dispatch
(``_module_linear``); a real model keeps its own parallel linears.  These
stand-ins carry the partition attributes the reference's layers expose
(H3/distributed/linear.py:36-191: ``input_size``, ``output_size``,
``tp_size``, ``tp_rank``, ``local_output_size`` / ``output_sizes`` +
``local_output_sizes`` / ``local_input_size``) and forward through the
dispatch, so the loader, the policies and the dispatch see the shape of
module tree they serve."""

from __future__ import annotations

from collections.abc import Sequence

import torch

import taomate_h3_amd.distributed.linear as dispatch


def _param(shape, dtype, device):
    return torch.nn.Parameter(torch.empty(shape, dtype=dtype, device=device))


class ToyColumnLinear(torch.nn.Module):
    """Rank ``tp_rank`` of ``tp_size``: output rows [rank * local, (rank + 1) * local)."""

    def __init__(self, in_features: int, out_features: int, *, bias: bool, dtype: torch.dtype,
                 tp: tuple[int, int] = (1, 0), device=None) -> None:
        super().__init__()
        self.tp_size, self.tp_rank = tp
        self.input_size, self.output_size = int(in_features), int(out_features)
        self.local_output_size = self.output_size // self.tp_size
        self.weight = _param((self.local_output_size, self.input_size), dtype, device)
        self.bias = _param((self.local_output_size,), dtype, device) if bias else None

    def forward(self, inputs: torch.Tensor) -> torch.Tensor:
        return dispatch._module_linear(self, inputs, self.bias)


class ToyMergedColumnLinear(ToyColumnLinear):
    """Several logical outputs (e.g. Q, K, V), each split over the ranks."""

    def __init__(self, in_features: int, out_features: Sequence[int], *, bias: bool, dtype: torch.dtype,
                 tp: tuple[int, int] = (1, 0), device=None) -> None:
        super().__init__(in_features, sum(out_features), bias=bias, dtype=dtype, tp=tp, device=device)
        self.output_sizes = tuple(int(v) for v in out_features)
        self.local_output_sizes = tuple(v // self.tp_size for v in self.output_sizes)


class ToyRowLinear(torch.nn.Module):
    """Rank ``tp_rank`` of ``tp_size``: input columns [rank * local, (rank + 1) * local);
    the output needs a cross-rank sum when tp_size > 1."""

    def __init__(self, in_features: int, out_features: int, *, bias: bool, dtype: torch.dtype,
                 tp: tuple[int, int] = (1, 0), device=None) -> None:
        super().__init__()
        self.tp_size, self.tp_rank = tp
        self.input_size, self.output_size = int(in_features), int(out_features)
        self.local_input_size = self.input_size // self.tp_size
        self.weight = _param((self.output_size, self.local_input_size), dtype, device)
        self.bias = _param((self.output_size,), dtype, device) if bias else None

    def forward_local(self, inputs: torch.Tensor) -> torch.Tensor:
        """This rank's partial output, without the bias."""
        return dispatch._module_linear(self, inputs, None)

    def reduce_local_output(self, value: torch.Tensor) -> torch.Tensor:
        if self.tp_size > 1:
            raise dispatch._cross_rank("reducing the output")
        return value

    def forward(self, inputs: torch.Tensor) -> torch.Tensor:
        out = self.reduce_local_output(self.forward_local(inputs))
        return out if self.bias is None else out + self.bias


class ToyReferenceLoRAWrapper(torch.nn.Module):
    """Stand-in for the wrapper class that the reference's
    ``apply_h3_lora_checkpoint`` defines inside the function and installs with
    ``setattr`` (H3/inference/lora_checkpoint.py:172-205, FL :440-489): the
    same attribute names, marker and buffers, and the same unfused forward
    (base, then two ``F.linear`` calls and the scaled add), single rank only."""

    def __init__(self, base, *, kind: str, a: torch.Tensor, b: torch.Tensor, scale: float,
                 marker: str = "_taomate_h3_inference_lora") -> None:
        super().__init__()
        self.base = base
        self.kind = kind
        self.scale = scale
        self.fused_row_reduce_enabled = False
        if marker == "_digitalhuman_h3_inference_lora":
            self.adapter_enabled = True
        setattr(self, marker, True)
        self.register_buffer("lora_a", a, persistent=False)
        self.register_buffer("lora_b", b, persistent=False)

    def forward(self, inputs: torch.Tensor) -> torch.Tensor:
        output = self.base(inputs)
        if not getattr(self, "adapter_enabled", True):
            return output
        compute_dtype = output.dtype
        update = torch.nn.functional.linear(
            torch.nn.functional.linear(inputs.to(compute_dtype), self.lora_a.to(compute_dtype)),
            self.lora_b.to(compute_dtype))
        return output + update * self.scale


def install_reference_lora(transformer: torch.nn.Module, targets, *, rank: int, scale: float, seed: int,
                           marker: str = "_taomate_h3_inference_lora") -> dict:
    """Install ToyReferenceLoRAWrapper on each named target the way the
    reference does (fp32 A [rank, K_local] and B [N_local, rank] buffers on the
    weight's device, then ``setattr`` on the parent); returns the wrappers."""
    gen = torch.Generator().manual_seed(seed)
    installed = {}
    for name in targets:
        module = transformer.get_submodule(name)
        n, k = (int(v) for v in module.weight.shape)
        kind = "row" if hasattr(module, "local_input_size") else "column"
        a = (torch.randn(rank, k, generator=gen) * 0.02).to(module.weight.device)
        b = (torch.randn(n, rank, generator=gen) * 0.02).to(module.weight.device)
        wrapper = ToyReferenceLoRAWrapper(module, kind=kind, a=a, b=b, scale=scale, marker=marker).eval()
        parent_name, _, leaf = name.rpartition(".")
        setattr(transformer.get_submodule(parent_name) if parent_name else transformer, leaf, wrapper)
        installed[name] = wrapper
    return installed
