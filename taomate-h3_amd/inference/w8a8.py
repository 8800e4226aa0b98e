"""Int8 W8A8 for the interior H3 projections on MI355X.

Drop-in for ``taomate_h3.inference.w8a8`` (H3/inference/w8a8.py:1-301): the
same names, module attributes, receipts and error messages, with the vLLM
CUDA operators replaced by the gfx950 library (include/taomate_h3_amd.h):

* ``require_vllm_cutlass_w8a8`` (w8a8.py:17-26) returns a backend object
  exposing vLLM's two allocating ops, ``scaled_int8_quant`` and
  ``cutlass_scaled_mm``, implemented by ``h3q_quant_rows`` (RCP_MUL) and
  ``h3q_scaled_mm``.
* ``_quantize_weight`` (w8a8.py:57-63) is ``h3q_quant_rows`` (INT8, DIV):
  bit-identical codes and scales, computed on the device.
* ``CutlassW8A8Workspace`` (w8a8.py:136-187) keeps the grow-only per
  (device, stream, width) buffers and the aliasing of same-width outputs.

Module state keeps the reference's names, shapes and byte counts:
``weight`` int8 ``[N, K]``, ``_cutlass_w8a8_weight_scale`` fp32 ``[N, 1]``
(non-persistent), the stream-load flags and the optional workspace views.
When N % 16 == 0 and K % 128 == 0 (every H3 projection) the codes in
``weight`` are stored in the GEMMs' tiled layout (16-row x 128-byte MFMA
fragment tiles, include/taomate_h3_amd.h), recorded against the parameter's
storage (``ops.is_tiled`` holds for the parameter and every view of it, such
as ``weight.t()``); otherwise they are row-major.  The tiled writer
quantizes straight into that layout, row chunk by row chunk.
"""

from __future__ import annotations

from collections.abc import Callable
from functools import lru_cache
from typing import Any

import torch

from .. import _lib, ops

INTERIOR_FC1_QKV_POLICY = "interior_fc1_qkv_v1"
_STREAM_LOAD_TEMPORARY_BYTES = 8 * 1024 * 1024


class NativeW8A8Backend:
    """vLLM's allocating W8A8 operators (``vllm._custom_ops``) on gfx950."""

    @staticmethod
    def scaled_int8_quant(input: torch.Tensor, scale: torch.Tensor | None = None, azp: torch.Tensor | None = None,
                          symmetric: bool = True) -> tuple[torch.Tensor, torch.Tensor, None]:
        """Dynamic per-token symmetric int8: (codes [M, K], scales [M, 1], None)."""
        if scale is not None or azp is not None or not symmetric:
            raise RuntimeError("only dynamic symmetric per-token int8 quantization is implemented")
        q, s = ops.quant_rows(input, ops.FMT_INT8, ops.ROUND_RCP_MUL)
        return q, s, None

    @staticmethod
    def cutlass_scaled_mm(a: torch.Tensor, b: torch.Tensor, scale_a: torch.Tensor, scale_b: torch.Tensor,
                          out_dtype: torch.dtype, bias: torch.Tensor | None = None) -> torch.Tensor:
        """bf16 ``scale_a * (scale_b * (a @ b))`` with ``b = weight.t()`` (a [K, N] column-major view)."""
        if out_dtype != torch.bfloat16:
            raise RuntimeError("cutlass_scaled_mm on gfx950 produces bfloat16 outputs")
        return ops.scaled_mm(a, b.t(), scale_a.reshape(-1), scale_b.reshape(-1), bias=bias)


@lru_cache(maxsize=1)
def require_vllm_cutlass_w8a8() -> Any:
    """Probe the native backend (the role of H3/inference/w8a8.py:17-26)."""
    try:
        _lib.lib()
    except (OSError, RuntimeError) as exc:
        raise RuntimeError("W8A8 requires the gfx950 quantized-linear library") from exc
    backend = NativeW8A8Backend()
    for name in ("scaled_int8_quant", "cutlass_scaled_mm"):
        if not callable(getattr(backend, name, None)):
            raise RuntimeError(f"gfx950 quantized-linear library is missing {name}")
    return backend


def resolve_h3_cutlass_w8a8_policy(names: list[str], *, policy: str) -> dict[str, Any]:
    """Select the fixed interior QKV/FC1 projection set (H3/inference/w8a8.py:29-54).

    Candidates are ``blocks.<i>.{attn.qkv_proj, mlp.fc1, mlp.fc2}``; the first
    two and last three candidate blocks stay BF16, and only QKV and FC1 of
    the remaining blocks are quantized."""
    if policy != INTERIOR_FC1_QKV_POLICY:
        raise ValueError(f"unsupported H3 W8A8 policy: {policy}")
    candidates = [n for n in names if n.startswith("blocks.") and n.endswith((".attn.qkv_proj", ".mlp.fc1",
                                                                               ".mlp.fc2"))]
    blocks = sorted({int(n.split(".", 2)[1]) for n in candidates})
    if not blocks:
        raise RuntimeError("H3 W8A8 found no DiT projections")
    protected = set(blocks[:2]) | set(blocks[-3:])
    selected = [n for n in candidates
                if n.endswith((".attn.qkv_proj", ".mlp.fc1")) and int(n.split(".", 2)[1]) not in protected]
    chosen = set(selected)
    return {
        "quantized_linear_names": selected,
        "bf16_protected_linear_names": [n for n in candidates if n not in chosen],
        "bf16_boundary_block_indices": sorted(protected),
    }


def _quantize_weight(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-output-channel int8 codes and fp32 scales of a bf16 weight (H3/inference/w8a8.py:57-63)."""
    return ops.quant_rows(weight, ops.FMT_INT8, ops.ROUND_DIV)


def prepare_cutlass_w8a8_stream_load_slot_(module: Any, *, name: str) -> None:
    """Replace one uninitialized BF16 parameter with its final W8 storage (H3/inference/w8a8.py:66-95)."""
    weight = module.weight
    if weight.dtype != torch.bfloat16:
        raise TypeError(f"{name} expected an uninitialized BF16 weight")
    if weight.requires_grad is False:
        raise RuntimeError(f"{name} uninitialized BF16 weight is already frozen")
    if module.bias is not None:
        raise RuntimeError(f"{name} expected a bias-free H3 projection")
    module.weight = torch.nn.Parameter(torch.empty(weight.shape, dtype=torch.int8, device=weight.device),
                                       requires_grad=False)
    if ops.can_tile(int(weight.shape[0]), int(weight.shape[1])):
        ops.mark_module_weight_tiled(module)
    module.register_buffer("_cutlass_w8a8_weight_scale",
                           torch.empty((int(weight.shape[0]), 1), dtype=torch.float32, device=weight.device),
                           persistent=False)
    module._cutlass_w8a8_stream_load_pending = True
    module._cutlass_w8a8_stream_loaded = False
    module._cutlass_w8a8_source_weight_bytes = int(weight.numel() * weight.element_size())


def load_cutlass_w8a8_stream_weight_(module: Any, source_weight: torch.Tensor, *, name: str,
                                     maximum_temporary_bytes: int = _STREAM_LOAD_TEMPORARY_BYTES) -> None:
    """Quantize a (CPU) BF16 checkpoint tensor into the module's device W8 storage
    in bounded row chunks (H3/inference/w8a8.py:98-133).  Scales are per row,
    so chunked quantization equals whole-matrix quantization; each chunk's
    codes and scales are written by the kernel straight into their final rows."""
    if getattr(module, "_cutlass_w8a8_stream_load_pending", None) is not True:
        raise RuntimeError(f"{name} has no pending CUTLASS W8A8 stream load")
    if module.weight.dtype != torch.int8 or source_weight.dtype != torch.bfloat16:
        raise TypeError(f"{name} streamed CUTLASS W8A8 dtype differs")
    if source_weight.ndim != 2 or tuple(source_weight.shape) != tuple(module.weight.shape):
        raise ValueError(f"{name} streamed CUTLASS W8A8 shape differs")
    stream_quantize_rows_(module, int(source_weight.shape[0]), int(source_weight.shape[1]),
                          lambda start, stop: source_weight[start:stop], name=name,
                          maximum_temporary_bytes=maximum_temporary_bytes)


def stream_quantize_rows_(module: Any, rows: int, cols: int, fetch: Callable[[int, int], torch.Tensor], *,
                          name: str, maximum_temporary_bytes: int = _STREAM_LOAD_TEMPORARY_BYTES) -> None:
    """Fill a pending W8 slot from a bf16 [rows, cols] matrix that ``fetch(start,
    stop)`` hands over in row ranges (a CPU or device tensor each; a streamed
    checkpoint reads them from disk on demand).

    Host rows go through two pinned staging buffers and two device buffers of
    ``maximum_temporary_bytes / 2`` each, so the fetch of one chunk overlaps
    the copy and quantization of the previous one, and the device staging
    stays within the bound the reference sets (H3/inference/w8a8.py:105-133)."""
    if getattr(module, "_cutlass_w8a8_stream_load_pending", None) is not True:
        raise RuntimeError(f"{name} has no pending CUTLASS W8A8 stream load")
    if maximum_temporary_bytes <= 0:
        raise ValueError("maximum_temporary_bytes must be positive")
    weight = module.weight
    scale = module._cutlass_w8a8_weight_scale
    if weight.dtype != torch.int8 or tuple(weight.shape) != (rows, cols):
        raise ValueError(f"{name} streamed CUTLASS W8A8 shape differs")
    device = weight.device
    tiled = ops.is_tiled(weight)
    rows_per_chunk = max(1, min(rows, (maximum_temporary_bytes // 2) // (cols * 2)))
    pinned: list[torch.Tensor | None] = [None, None]
    staged = [torch.empty((rows_per_chunk, cols), dtype=torch.bfloat16, device=device) for _ in range(2)]
    released: list[torch.cuda.Event | None] = [None, None]
    stream = torch.cuda.current_stream(device)
    for i, start in enumerate(range(0, rows, rows_per_chunk)):
        stop = min(start + rows_per_chunk, rows)
        n, b = stop - start, i % 2
        chunk = fetch(start, stop)
        if chunk.dtype != torch.bfloat16 or tuple(chunk.shape) != (n, cols):
            raise ValueError(f"{name} streamed rows [{start}, {stop}) are not bf16 [{n}, {cols}]")
        if chunk.device.type == "cpu":
            if released[b] is not None:
                released[b].synchronize()  # the copy that last read this pinned buffer is done
            if pinned[b] is None:
                pinned[b] = torch.empty((rows_per_chunk, cols), dtype=torch.bfloat16, pin_memory=True)
            pinned[b][:n].copy_(chunk)
            staged[b][:n].copy_(pinned[b][:n], non_blocking=True)
            source = staged[b][:n]
        else:
            source = chunk.to(device=device)
        if tiled:
            ops.quant_rows_tiled(source, ops.FMT_INT8, ops.ROUND_DIV, codes=weight.data, row0=start,
                                 scales=scale[start:stop])
        else:
            ops.quant_rows(source, ops.FMT_INT8, ops.ROUND_DIV, codes=weight.data[start:stop],
                           scales=scale[start:stop])
        released[b] = torch.cuda.Event()
        released[b].record(stream)
    for event in released:
        if event is not None:
            event.synchronize()
    module._cutlass_w8a8_stream_load_temporary_bytes_limit = int(maximum_temporary_bytes)
    module._cutlass_w8a8_stream_load_pending = False
    module._cutlass_w8a8_stream_loaded = True


class CutlassW8A8Workspace:
    """Grow-only per-stream buffers shared by serial H3 QKV/FC1 calls
    (H3/inference/w8a8.py:136-187).

    Activation codes/scales are keyed by (device, stream, K) and outputs by
    (device, stream, N); calls return views ``[:M]``.  Two calls with the same
    output width on the same stream return the same storage, so a caller must
    consume an output before the next same-width call, exactly as with the
    reference."""

    def __init__(self) -> None:
        require_vllm_cutlass_w8a8()
        self._activation: dict[tuple[int | None, int, int], tuple[torch.Tensor, torch.Tensor]] = {}
        self._outputs: dict[tuple[int | None, int, int], torch.Tensor] = {}

    @staticmethod
    def _stream(inputs: torch.Tensor) -> tuple[int | None, int]:
        stream = torch.cuda.current_stream(device=inputs.device)
        return inputs.device.index, int(stream.cuda_stream)

    def buffers(self, inputs: torch.Tensor, output_width: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """(codes [M, K] int8, scales [M, 1] fp32, out [M, N] bf16) views for this call.
        The codes buffer holds at least ops.tiled_rows(M) rows (the tiled
        layout pads to 16); ``_codes_buffer`` returns it whole."""
        rows, width = int(inputs.shape[0]), int(inputs.shape[1])
        device_index, stream = self._stream(inputs)
        key = (device_index, stream, width)
        act = self._activation.get(key)
        if act is None or int(act[1].shape[0]) < rows:
            act = (torch.empty((ops.tiled_rows(rows), width), device=inputs.device, dtype=torch.int8),
                   torch.empty((rows, 1), device=inputs.device, dtype=torch.float32))
            self._activation[key] = act
        out_key = (device_index, stream, int(output_width))
        out = self._outputs.get(out_key)
        if out is None or int(out.shape[0]) < rows:
            out = torch.empty((rows, int(output_width)), device=inputs.device, dtype=torch.bfloat16)
            self._outputs[out_key] = out
        return act[0][:rows], act[1][:rows], out[:rows]

    def _codes_buffer(self, inputs: torch.Tensor) -> torch.Tensor:
        device_index, stream = self._stream(inputs)
        return self._activation[(device_index, stream, int(inputs.shape[1]))][0]

    def linear(self, inputs: torch.Tensor, weight_t: torch.Tensor, weight_scale_t: torch.Tensor) -> torch.Tensor:
        rows = int(inputs.shape[0])
        _, activation_scale, output = self.buffers(inputs, int(weight_t.shape[1]))
        quantized, activation_scale, a_tiled = ops.quant_activations_for(
            inputs, ops.FMT_INT8, ops.ROUND_RCP_MUL, weight_t, codes=self._codes_buffer(inputs),
            scales=activation_scale)
        ops.scaled_mm(quantized, weight_t.t(), activation_scale, weight_scale_t.reshape(-1), out=output,
                      a_tiled=a_tiled, b_tiled=ops.is_tiled(weight_t), m=rows)
        return output


def cutlass_w8a8_linear(inputs: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor, *,
                        bias: torch.Tensor | None, workspace: CutlassW8A8Workspace | None,
                        weight_t: torch.Tensor | None, weight_scale_t: torch.Tensor | None) -> torch.Tensor:
    """Dynamic per-token int8 activations x per-channel int8 weights -> bf16
    (H3/inference/w8a8.py:190-220)."""
    if bias is not None:
        raise RuntimeError("H3 W8A8 supports bias-free linears only")
    from .fused_kernels import QuantizedActivations

    if isinstance(inputs, QuantizedActivations):
        return _linear_from_codes(inputs, weight, weight_scale, workspace)
    shape = (*inputs.shape[:-1], int(weight.shape[0]))
    flattened = inputs.reshape(-1, int(inputs.shape[-1])).contiguous()
    if workspace is not None:
        if weight_t is None:
            weight_t = weight.t()
        output = workspace.linear(flattened, weight_t, weight_scale.t() if weight_scale_t is None else weight_scale_t)
        return output.reshape(shape)
    if ops.is_tiled(weight):
        quantized, activation_scale, a_tiled = ops.quant_activations_for(flattened, ops.FMT_INT8, ops.ROUND_RCP_MUL,
                                                                         weight)
        output = ops.scaled_mm(quantized, weight, activation_scale.reshape(-1), weight_scale.reshape(-1),
                               a_tiled=a_tiled, b_tiled=True, m=int(flattened.shape[0]))
        return output.reshape(shape)
    backend = require_vllm_cutlass_w8a8()
    quantized, activation_scale, _ = backend.scaled_int8_quant(flattened)
    output = backend.cutlass_scaled_mm(quantized, weight.t(), activation_scale, weight_scale.t(), torch.bfloat16)
    return output.reshape(shape)


def _linear_from_codes(inputs: Any, weight: torch.Tensor, weight_scale: torch.Tensor,
                       workspace: CutlassW8A8Workspace | None) -> torch.Tensor:
    """The W8A8 GEMM on activations already quantized per token (int8, vLLM
    form) by a fused producer: the act-quant pass of the linear is skipped."""
    if inputs.fmt != ops.FMT_INT8 or inputs.codes.dtype != torch.int8:
        raise TypeError("H3 W8A8 linear expects int8 activation codes")
    rows = int(inputs.codes.shape[0])
    shape = (*inputs.shape[:-1], int(weight.shape[0]))
    out = None
    if workspace is not None:
        _, _, out = workspace.buffers(inputs.codes, int(weight.shape[0]))
    output = ops.scaled_mm(inputs.codes, weight, inputs.scales.reshape(-1), weight_scale.reshape(-1), out=out,
                           b_tiled=ops.is_tiled(weight), m=rows)
    return output.reshape(shape)


def _projection_candidates(transformer: Any) -> list[tuple[str, Any]]:
    """DiT projections eligible for W8A8: LoRA wrappers contribute their frozen ``base``."""
    found = []
    for name, module in transformer.named_modules():
        if not name.startswith("blocks.") or not name.endswith((".attn.qkv_proj", ".mlp.fc1", ".mlp.fc2")):
            continue
        base = getattr(module, "base", module)
        weight = getattr(base, "weight", None)
        if isinstance(base, torch.nn.Module) and isinstance(weight, torch.Tensor) and weight.ndim == 2:
            found.append((name, base))
    return found


def quantize_h3_interior_qkv_fc1_(transformer: Any, *, policy: str) -> dict[str, Any]:
    """Validate and summarize the streamed base W8A8 linears (H3/inference/w8a8.py:223-268)."""
    require_vllm_cutlass_w8a8()
    candidates = _projection_candidates(transformer)
    selection = resolve_h3_cutlass_w8a8_policy([n for n, _ in candidates], policy=policy)
    selected = set(selection["quantized_linear_names"])
    chosen = [(n, m) for n, m in candidates if n in selected]
    if not chosen:
        raise RuntimeError("H3 W8A8 policy selected no linears")
    source_bytes = quantized_bytes = 0
    for name, module in chosen:
        scale = getattr(module, "_cutlass_w8a8_weight_scale", None)
        if (scale is None or module.weight.dtype != torch.int8
                or getattr(module, "_cutlass_w8a8_stream_load_pending", None) is not False
                or getattr(module, "_cutlass_w8a8_stream_loaded", None) is not True):
            raise RuntimeError(f"{name} was not loaded directly as CUTLASS W8A8")
        if module.bias is not None:
            raise RuntimeError(f"{name} is not a bias-free projection")
        source_bytes += int(module._cutlass_w8a8_source_weight_bytes)
        quantized_bytes += int(module.weight.numel() * module.weight.element_size())
    return {
        "policy": policy,
        "format": "int8_w8a8",
        "linear_count": len(chosen),
        "stream_load_linear_count": len(chosen),
        "post_load_conversion_linear_count": 0,
        "source_weight_bytes": source_bytes,
        "quantized_weight_bytes": quantized_bytes,
        **selection,
    }


def enable_h3_cutlass_w8a8_workspace_(transformer: Any) -> dict[str, Any]:
    """Attach one shared workspace and the transposed views (H3/inference/w8a8.py:271-289)."""
    require_vllm_cutlass_w8a8()
    selected = [m for m in transformer.modules() if getattr(m, "_cutlass_w8a8_weight_scale", None) is not None]
    if not selected:
        raise RuntimeError("W8A8 workspace requires quantized H3 linears")
    workspace = CutlassW8A8Workspace()
    for module in selected:
        module._cutlass_w8a8_workspace = workspace
        module._cutlass_w8a8_weight_t = module.weight.t()
        module._cutlass_w8a8_weight_scale_t = module._cutlass_w8a8_weight_scale.t()
    return {
        "linear_count": len(selected),
        "workspace_count_per_rank": 1,
        "allocation_policy": "grow_only_per_cuda_stream_and_shape",
    }


__all__ = [
    "INTERIOR_FC1_QKV_POLICY",
    "CutlassW8A8Workspace",
    "NativeW8A8Backend",
    "cutlass_w8a8_linear",
    "enable_h3_cutlass_w8a8_workspace_",
    "load_cutlass_w8a8_stream_weight_",
    "prepare_cutlass_w8a8_stream_load_slot_",
    "quantize_h3_interior_qkv_fc1_",
    "require_vllm_cutlass_w8a8",
    "resolve_h3_cutlass_w8a8_policy",
    "stream_quantize_rows_",
]
