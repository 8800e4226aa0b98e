"""Streamed checkpoint loading into TP-local and quantized parameters:
H3/model/weight_loading.py:29-264 with the W8 slots of
H3/inference/w8a8.py:66-133.

Same names, checks, errors and receipt as the reference
(``load_minimax_h3_dit_weights``, ``reorder_grouped_qkv_to_qkv``,
``H3NativeWeightError``).  The difference is how a pending W8 slot is filled.
The reference reads the whole bf16 tensor, reorders and slices it on the host,
then quantizes 8 MiB row chunks on the GPU.  Here every destination row of the
rank's shard is mapped back to its checkpoint row (the grouped-QKV reorder and
the TP slice compose into one row map plus a column range), and the rows are
read from the safetensors file range by range (``get_slice``), staged through
pinned memory and quantized straight into their tiled positions.  Neither the
full tensor nor its reordered copy is ever materialized.  Scales are per row,
so the codes equal those of the reference's whole-tensor path bit for bit.

The model may be any ``nn.Module`` whose state dict names match the checkpoint;
the QKV reorder reads ``model.arch.num_attention_heads`` and
``model.arch.attention_head_dim`` as the reference does.
"""

from __future__ import annotations

import importlib
import json
from collections.abc import Mapping
from pathlib import Path
from typing import Any

import torch

from .distributed.linear import ColumnParallelLinear, MergedColumnParallelLinear, RowParallelLinear
from .inference.w8a8 import _STREAM_LOAD_TEMPORARY_BYTES, stream_quantize_rows_


class H3NativeWeightError(RuntimeError):
    pass


def qkv_row_order(*, num_query_groups: int, heads_per_group: int, head_dim: int) -> torch.Tensor:
    """Checkpoint row of every output row of ``reorder_grouped_qkv_to_qkv``:
    groups of (heads_per_group query heads, one key head, one value head)
    become all query rows, then all key rows, then all value rows."""
    per_group = (heads_per_group + 2) * head_dim
    q_rows = heads_per_group * head_dim
    g = torch.arange(num_query_groups).view(-1, 1)
    q = (g * per_group + torch.arange(q_rows).view(1, -1)).reshape(-1)
    k = (g * per_group + q_rows + torch.arange(head_dim).view(1, -1)).reshape(-1)
    v = (g * per_group + q_rows + head_dim + torch.arange(head_dim).view(1, -1)).reshape(-1)
    return torch.cat((q, k, v))


def reorder_grouped_qkv_to_qkv(weight: torch.Tensor, *, num_query_groups: int, heads_per_group: int,
                               head_dim: int) -> torch.Tensor:
    """H3/model/weight_loading.py:29-54."""
    per_group = (heads_per_group + 2) * head_dim
    if int(weight.shape[0]) != num_query_groups * per_group:
        raise H3NativeWeightError("qkv checkpoint rows differ from grouped MiniMax H3 layout")
    order = qkv_row_order(num_query_groups=num_query_groups, heads_per_group=heads_per_group, head_dim=head_dim)
    return weight.index_select(0, order.to(weight.device))


def _safe_regular_root(path: Path) -> Path:
    try:
        root = path.expanduser().resolve(strict=True)
    except OSError as exc:
        raise H3NativeWeightError(f"cannot resolve H3 transformer root: {exc}") from exc
    if not root.is_dir():
        raise H3NativeWeightError("H3 transformer root must be a directory")
    return root


def _index_weight_map(root: Path) -> Mapping[str, str] | None:
    """H3/model/weight_loading.py:67-88."""
    candidates = (root / "diffusion_pytorch_model.safetensors.index.json", root / "model.safetensors.index.json")
    existing = [path for path in candidates if path.is_file()]
    if len(existing) > 1:
        raise H3NativeWeightError("multiple H3 safetensors index files are present")
    if not existing:
        return None
    try:
        payload = json.loads(existing[0].read_text(encoding="utf-8"))
    except (OSError, UnicodeError, json.JSONDecodeError) as exc:
        raise H3NativeWeightError(f"cannot read H3 safetensors index: {exc}") from exc
    weight_map = payload.get("weight_map") if isinstance(payload, Mapping) else None
    if not isinstance(weight_map, Mapping) or not weight_map:
        raise H3NativeWeightError("H3 safetensors index weight_map is absent")
    if any(not isinstance(k, str) or not isinstance(v, str) for k, v in weight_map.items()):
        raise H3NativeWeightError("H3 safetensors index contains non-string entries")
    return dict(weight_map)


def _resolve_shards(root: Path) -> tuple[dict[str, Path], tuple[Path, ...]]:
    """H3/model/weight_loading.py:91-122."""
    weight_map = _index_weight_map(root)
    if weight_map is None:
        shards = tuple(sorted(root.glob("*.safetensors")))
        if not shards:
            raise H3NativeWeightError("H3 transformer safetensors are absent")
        safe_open = importlib.import_module("safetensors").safe_open
        resolved: dict[str, Path] = {}
        canonical = tuple(shard.resolve(strict=True) for shard in shards)
        for shard in canonical:
            if not shard.is_file():
                raise H3NativeWeightError("H3 safetensors shard must be a file")
            with safe_open(str(shard), framework="pt", device="cpu") as handle:
                for key in handle.keys():
                    if key in resolved:
                        raise H3NativeWeightError(f"duplicate H3 tensor key: {key}")
                    resolved[key] = shard
        return resolved, canonical
    by_filename: dict[str, Path] = {}
    for filename in sorted(set(weight_map.values())):
        relative = Path(filename)
        if relative.is_absolute() or ".." in relative.parts:
            raise H3NativeWeightError("H3 safetensors index escapes transformer root")
        try:
            candidate = (root / relative).resolve(strict=True)
        except OSError as exc:
            raise H3NativeWeightError(f"H3 safetensors shard is absent: {filename}") from exc
        if not candidate.is_file():
            raise H3NativeWeightError(f"H3 safetensors shard is absent: {filename}")
        by_filename[filename] = candidate
    return {key: by_filename[value] for key, value in weight_map.items()}, tuple(by_filename.values())


def _qkv_reorder_args(model: Any) -> dict[str, int]:
    arch = getattr(model, "arch", None)
    heads = getattr(arch, "num_attention_heads", None)
    head_dim = getattr(arch, "attention_head_dim", None)
    if not isinstance(heads, int) or not isinstance(head_dim, int):
        raise H3NativeWeightError("the QKV reorder needs model.arch.num_attention_heads and attention_head_dim")
    return {"num_query_groups": heads, "heads_per_group": 1, "head_dim": head_dim}


def _local_tensor(name: str, value: torch.Tensor, *, owner: torch.nn.Module, leaf: str, model: Any) -> torch.Tensor:
    """H3/model/weight_loading.py:125-151: the rank's slice of a full tensor."""
    if isinstance(owner, MergedColumnParallelLinear):
        if leaf not in {"weight", "bias"}:
            return value
        if name.endswith("attn.qkv_proj.weight"):
            value = reorder_grouped_qkv_to_qkv(value, **_qkv_reorder_args(model))
        return owner.full_weight_slice(value) if leaf == "weight" else owner.full_bias_slice(value)
    if isinstance(owner, ColumnParallelLinear):
        if leaf == "weight":
            return owner.full_weight_slice(value)
        if leaf == "bias":
            return owner.full_bias_slice(value)
    if isinstance(owner, RowParallelLinear) and leaf == "weight":
        return owner.full_weight_slice(value)
    return value


def _local_weight_map(name: str, full_shape: tuple[int, ...], *, owner: torch.nn.Module,
                      model: Any) -> tuple[torch.Tensor, int, int]:
    """The same slice as ``_local_tensor`` for a weight, as (checkpoint row of
    each local row, first column, column count), checked against the owner's
    expected full shape."""
    rows, cols = int(full_shape[0]), int(full_shape[1])
    row_map = torch.arange(rows)
    if isinstance(owner, MergedColumnParallelLinear):
        if name.endswith("attn.qkv_proj.weight"):
            args = _qkv_reorder_args(model)
            if rows != args["num_query_groups"] * (args["heads_per_group"] + 2) * args["head_dim"]:
                raise H3NativeWeightError("qkv checkpoint rows differ from grouped MiniMax H3 layout")
            row_map = qkv_row_order(**args)
        if (rows, cols) != (owner.output_size, owner.input_size):
            raise ValueError("full merged-column weight shape differs")
        pieces, offset = [], 0
        for size, local in zip(owner.output_sizes, owner.local_output_sizes):
            pieces.append(row_map[offset + owner.tp_rank * local: offset + (owner.tp_rank + 1) * local])
            offset += size
        return torch.cat(pieces), 0, cols
    if isinstance(owner, ColumnParallelLinear):
        if (rows, cols) != (owner.output_size, owner.input_size):
            raise ValueError("full column-parallel weight shape differs")
        local = owner.local_output_size
        return row_map[owner.tp_rank * local:(owner.tp_rank + 1) * local], 0, cols
    if isinstance(owner, RowParallelLinear):
        if (rows, cols) != (owner.output_size, owner.input_size):
            raise ValueError("full row-parallel weight shape differs")
        return row_map, owner.tp_rank * owner.local_input_size, owner.local_input_size
    return row_map, 0, cols


def _row_runs(rows: torch.Tensor) -> list[tuple[int, int, int]]:
    """(destination offset, first checkpoint row, count) of each run of
    consecutive checkpoint rows."""
    values = rows.tolist()
    runs, start = [], 0
    for i in range(1, len(values) + 1):
        if i == len(values) or values[i] != values[i - 1] + 1:
            runs.append((start, values[start], i - start))
            start = i
    return runs


def _stream_w8a8_slot(owner: Any, name: str, handle: Any, *, model: Any, maximum_temporary_bytes: int) -> None:
    """Fill a pending W8 slot from the checkpoint, reading only the rank's rows."""
    source = handle.get_slice(name)
    dtype = source.get_dtype()
    if dtype not in ("BF16", "bfloat16"):
        raise TypeError(f"{name} streamed CUTLASS W8A8 dtype differs")
    full_shape = tuple(int(v) for v in source.get_shape())
    if len(full_shape) != 2:
        raise H3NativeWeightError(f"H3 local tensor shape differs for {name}: {full_shape}")
    row_map, col0, ncols = _local_weight_map(name, full_shape, owner=owner, model=model)
    local_shape = (int(row_map.numel()), ncols)
    if local_shape != tuple(owner.weight.shape):
        raise H3NativeWeightError(f"H3 local tensor shape differs for {name}: {local_shape} != "
                                  f"{tuple(owner.weight.shape)}")
    runs = _row_runs(row_map)

    def fetch(start: int, stop: int) -> torch.Tensor:
        parts = []
        for dst, src, count in runs:
            lo, hi = max(dst, start), min(dst + count, stop)
            if lo < hi:
                parts.append(source[src + lo - dst: src + hi - dst, col0: col0 + ncols])
        return parts[0] if len(parts) == 1 else torch.cat(parts)

    stream_quantize_rows_(owner, local_shape[0], ncols, fetch, name=name,
                          maximum_temporary_bytes=maximum_temporary_bytes)


def load_minimax_h3_dit_weights(model: torch.nn.Module, transformer_root: str | Path, *,
                                maximum_temporary_bytes: int = _STREAM_LOAD_TEMPORARY_BYTES) -> dict[str, Any]:
    """Stream safetensors one tensor at a time into TP-local parameters
    (H3/model/weight_loading.py:154-264); pending W8 slots are filled by
    row-range reads quantized on the device."""
    if not isinstance(model, torch.nn.Module):
        raise TypeError("model must be an nn.Module")
    root = _safe_regular_root(Path(transformer_root))
    key_to_shard, shards = _resolve_shards(root)
    safe_open = importlib.import_module("safetensors").safe_open
    state = model.state_dict(keep_vars=True)
    expected, present = set(state), set(key_to_shard)
    missing, unexpected = sorted(expected - present), sorted(present - expected)
    if missing or unexpected:
        raise H3NativeWeightError("H3 transformer tensor inventory differs: "
                                  f"missing={missing[:8]}, unexpected={unexpected[:8]}")
    modules = dict(model.named_modules())
    by_shard: dict[Path, list[str]] = {path: [] for path in shards}
    for name, path in key_to_shard.items():
        by_shard[path].append(name)
    streamed_names: list[str] = []
    source_bytes = quantized_bytes = scale_bytes = temporary_limit = bf16_copies = 0
    with torch.no_grad():
        for shard in shards:
            with safe_open(str(shard), framework="pt", device="cpu") as handle:
                for name in sorted(by_shard[shard]):
                    destination = state[name]
                    owner_name, separator, leaf = name.rpartition(".")
                    if not separator:
                        owner_name, leaf = "", name
                    owner = modules.get(owner_name)
                    if owner is None:
                        raise H3NativeWeightError(f"H3 state owner is absent: {name}")
                    if leaf == "weight" and getattr(owner, "_cutlass_w8a8_stream_load_pending", None) is True:
                        _stream_w8a8_slot(owner, name, handle, model=model,
                                          maximum_temporary_bytes=maximum_temporary_bytes)
                        streamed_names.append(owner_name)
                        source_bytes += int(owner._cutlass_w8a8_source_weight_bytes)
                        quantized_bytes += int(owner.weight.numel() * owner.weight.element_size())
                        scale_bytes += int(owner._cutlass_w8a8_weight_scale.numel()
                                           * owner._cutlass_w8a8_weight_scale.element_size())
                        temporary_limit = max(temporary_limit,
                                              int(owner._cutlass_w8a8_stream_load_temporary_bytes_limit))
                        continue
                    value = _local_tensor(name, handle.get_tensor(name), owner=owner, leaf=leaf, model=model)
                    if tuple(value.shape) != tuple(destination.shape):
                        raise H3NativeWeightError(f"H3 local tensor shape differs for {name}: "
                                                  f"{tuple(value.shape)} != {tuple(destination.shape)}")
                    if value.dtype != destination.dtype:
                        raise H3NativeWeightError(f"H3 tensor dtype differs for {name}: "
                                                  f"{value.dtype} != {destination.dtype}")
                    destination.copy_(value)
                    if leaf == "weight" and value.dtype == torch.bfloat16:
                        bf16_copies += 1
    pending = [name for name, module in model.named_modules()
               if getattr(module, "_cutlass_w8a8_stream_load_pending", None) is True]
    if pending:
        raise H3NativeWeightError(f"H3 streamed W8A8 weights were not loaded: {pending[:8]}")
    receipt = {
        "shard_count": len(shards),
        "tensor_count": len(state),
        "stream_load_policy": getattr(model, "_load_time_w8a8_policy", None),
        "streamed_w8a8_linear_count": len(streamed_names),
        "streamed_w8a8_source_weight_bytes": source_bytes,
        "streamed_w8a8_quantized_weight_bytes": quantized_bytes,
        "streamed_w8a8_scale_bytes": scale_bytes,
        "stream_load_bf16_staging_bytes_limit": temporary_limit,
        "bf16_weight_copy_count": bf16_copies,
    }
    model._native_weight_load_receipt = receipt
    return receipt


__all__ = ["H3NativeWeightError", "load_minimax_h3_dit_weights", "qkv_row_order", "reorder_grouped_qkv_to_qkv"]
