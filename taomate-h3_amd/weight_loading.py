"""Streamed checkpoint loading into TP-local and quantized parameters.

Drop-in for ``load_minimax_h3_dit_weights`` and ``reorder_grouped_qkv_to_qkv``
(H3/model/weight_loading.py:29-264), with the W8 slots of
H3/inference/w8a8.py:66-133 filled on the device.  The error types and
messages and the receipt keys are the reference's; the loading itself is
planned differently:

* Every destination tensor gets a *placement*: the checkpoint row behind
  each of its local rows (the grouped-QKV reorder and the tensor-parallel
  slice of the owning module composed into one row map) and the column range
  of a row-parallel slice.  The owner's partition is read from the attributes
  the reference's parallel linears carry (``tp_rank``, ``output_sizes`` /
  ``local_output_sizes``, ``local_output_size``, ``local_input_size``), so any
  module tree with the reference's layer types and names loads.
* Rows are read from the safetensors file range by range (``get_slice``), so
  neither a full tensor nor its reordered copy is materialised.  bf16 rows
  are copied into their parameter; the rows of a pending W8 slot are staged
  through pinned memory and quantized on the device straight into their tiled
  positions (``stream_quantize_rows_``).  Scales are per row, so the codes
  equal those of the reference's whole-tensor path bit for bit.
* After loading, parameters and buffers that must stay fp32 are checked
  (H3/model/weight_loading.py:246-251): by default the name sets
  ``MINIMAX_H3_FP32_PARAM_NAMES`` / ``MINIMAX_H3_FP32_BUFFER_NAMES`` of the
  module that defines the model's class, or the sets passed in.
"""

from __future__ import annotations

import importlib
import json
import sys
from collections.abc import Iterable, Mapping
from dataclasses import dataclass
from pathlib import Path
from typing import Any

import torch

from .inference.w8a8 import _STREAM_LOAD_TEMPORARY_BYTES, stream_quantize_rows_

_INDEX_FILES = ("diffusion_pytorch_model.safetensors.index.json", "model.safetensors.index.json")


class H3NativeWeightError(RuntimeError):
    pass


# ----------------------------------------------------------------- QKV order

def qkv_row_order(*, num_query_groups: int, heads_per_group: int, head_dim: int) -> torch.Tensor:
    """Checkpoint row of every output row of ``reorder_grouped_qkv_to_qkv``:
    the checkpoint stores per group (heads_per_group query heads, one key
    head, one value head); the model wants all query rows, then all key
    rows, then all value rows."""
    per_group = (heads_per_group + 2) * head_dim
    q_rows = heads_per_group * head_dim
    starts = torch.arange(num_query_groups).view(-1, 1) * per_group
    q = (starts + torch.arange(q_rows)).reshape(-1)
    k = (starts + q_rows + torch.arange(head_dim)).reshape(-1)
    v = (starts + q_rows + head_dim + torch.arange(head_dim)).reshape(-1)
    return torch.cat((q, k, v))


def reorder_grouped_qkv_to_qkv(weight: torch.Tensor, *, num_query_groups: int, heads_per_group: int,
                               head_dim: int) -> torch.Tensor:
    """Grouped per-head QKV rows -> [Q; K; V] (H3/model/weight_loading.py:29-54)."""
    if int(weight.shape[0]) != num_query_groups * (heads_per_group + 2) * head_dim:
        raise H3NativeWeightError("qkv checkpoint rows differ from grouped MiniMax H3 layout")
    order = qkv_row_order(num_query_groups=num_query_groups, heads_per_group=heads_per_group, head_dim=head_dim)
    return weight.index_select(0, order.to(weight.device))


# ---------------------------------------------------------- checkpoint index

class _Checkpoint:
    """Where each tensor of a transformer directory lives: an index file's
    ``weight_map`` when one is present (H3/model/weight_loading.py:67-122), else
    the keys found in the directory's ``*.safetensors`` files."""

    def __init__(self, path: Path) -> None:
        try:
            self.root = path.expanduser().resolve(strict=True)
        except OSError as exc:
            raise H3NativeWeightError(f"cannot resolve H3 transformer root: {exc}") from exc
        if not self.root.is_dir():
            raise H3NativeWeightError("H3 transformer root must be a directory")
        indexes = [self.root / name for name in _INDEX_FILES if (self.root / name).is_file()]
        if len(indexes) > 1:
            raise H3NativeWeightError("multiple H3 safetensors index files are present")
        self.location = self._read_index(indexes[0]) if indexes else self._scan()
        self.shards = tuple(dict.fromkeys(sorted(self.location.values())))

    def _read_index(self, index: Path) -> dict[str, Path]:
        try:
            payload = json.loads(index.read_text(encoding="utf-8"))
        except (OSError, UnicodeError, json.JSONDecodeError) as exc:
            raise H3NativeWeightError(f"cannot read H3 safetensors index: {exc}") from exc
        entries = payload.get("weight_map") if isinstance(payload, Mapping) else None
        if not isinstance(entries, Mapping) or not entries:
            raise H3NativeWeightError("H3 safetensors index weight_map is absent")
        if not all(isinstance(k, str) and isinstance(v, str) for k, v in entries.items()):
            raise H3NativeWeightError("H3 safetensors index contains non-string entries")
        files: dict[str, Path] = {}
        for filename in sorted(set(entries.values())):
            relative = Path(filename)
            if relative.is_absolute() or ".." in relative.parts:
                raise H3NativeWeightError("H3 safetensors index escapes transformer root")
            try:
                shard = (self.root / relative).resolve(strict=True)
            except OSError as exc:
                raise H3NativeWeightError(f"H3 safetensors shard is absent: {filename}") from exc
            if not shard.is_file():
                raise H3NativeWeightError(f"H3 safetensors shard is absent: {filename}")
            files[filename] = shard
        return {key: files[filename] for key, filename in entries.items()}

    def _scan(self) -> dict[str, Path]:
        found = sorted(self.root.glob("*.safetensors"))
        if not found:
            raise H3NativeWeightError("H3 transformer safetensors are absent")
        safe_open = importlib.import_module("safetensors").safe_open
        location: dict[str, Path] = {}
        for shard in (p.resolve(strict=True) for p in found):
            if not shard.is_file():
                raise H3NativeWeightError("H3 safetensors shard must be a file")
            with safe_open(str(shard), framework="pt", device="cpu") as handle:
                for key in handle.keys():
                    if key in location:
                        raise H3NativeWeightError(f"duplicate H3 tensor key: {key}")
                    location[key] = shard
        return location


# ----------------------------------------------------------------- placement

@dataclass
class _Placement:
    """The local tensor as a selection of the full checkpoint tensor: rows
    ``rows[i]`` (None: all rows in order), columns [col0, col0 + ncols)
    (ncols None: all columns)."""

    rows: torch.Tensor | None = None
    col0: int = 0
    ncols: int | None = None

    def runs(self, total_rows: int) -> list[tuple[int, int, int]]:
        """(local row, checkpoint row, count) of each run of consecutive rows."""
        if self.rows is None:
            return [(0, 0, total_rows)]
        values = self.rows.tolist()
        out, start = [], 0
        for i in range(1, len(values) + 1):
            if i == len(values) or values[i] != values[i - 1] + 1:
                out.append((start, values[start], i - start))
                start = i
        return out


def _qkv_args(model: Any) -> dict[str, int]:
    arch = getattr(model, "arch", None)
    heads = getattr(arch, "num_attention_heads", None)
    head_dim = getattr(arch, "attention_head_dim", None)
    if not isinstance(heads, int) or not isinstance(head_dim, int):
        raise H3NativeWeightError("the QKV reorder needs model.arch.num_attention_heads and attention_head_dim")
    return {"num_query_groups": heads, "heads_per_group": 1, "head_dim": head_dim}


def _placement(name: str, leaf: str, full_shape: tuple[int, ...], owner: Any, model: Any) -> _Placement:
    """Placement of ``owner.<leaf>`` (checkpoint tensor ``name`` of ``full_shape``)
    on this rank, from the owner's partition attributes."""
    if leaf not in ("weight", "bias"):
        return _Placement()
    rank = int(getattr(owner, "tp_rank", 0))
    pieces = getattr(owner, "output_sizes", None)
    if pieces is not None:                                       # merged column-parallel
        out_rows = int(sum(pieces))
        if leaf == "weight" and tuple(full_shape) != (out_rows, int(owner.input_size)):
            raise ValueError("full merged-column weight shape differs")
        order = torch.arange(int(full_shape[0]))
        if name.endswith("attn.qkv_proj.weight"):
            args = _qkv_args(model)
            if int(full_shape[0]) != args["num_query_groups"] * (args["heads_per_group"] + 2) * args["head_dim"]:
                raise H3NativeWeightError("qkv checkpoint rows differ from grouped MiniMax H3 layout")
            order = qkv_row_order(**args)
        chosen, first = [], 0
        for size, local in zip(pieces, owner.local_output_sizes):
            chosen.append(order[first + rank * int(local): first + (rank + 1) * int(local)])
            first += int(size)
        return _Placement(rows=torch.cat(chosen))
    local_out = getattr(owner, "local_output_size", None)
    if local_out is not None:                                    # column-parallel
        if leaf == "weight" and tuple(full_shape) != (int(owner.output_size), int(owner.input_size)):
            raise ValueError("full column-parallel weight shape differs")
        return _Placement(rows=torch.arange(rank * int(local_out), (rank + 1) * int(local_out)))
    local_in = getattr(owner, "local_input_size", None)
    if local_in is not None and leaf == "weight":                # row-parallel: a column slice
        if tuple(full_shape) != (int(owner.output_size), int(owner.input_size)):
            raise ValueError("full row-parallel weight shape differs")
        return _Placement(col0=rank * int(local_in), ncols=int(local_in))
    return _Placement()


def _read_rows(source: Any, full_shape: tuple[int, ...], place: _Placement, start: int, stop: int) -> torch.Tensor:
    """Local rows [start, stop) of a 2-D (or 1-D) checkpoint tensor, read range by range."""
    cols = slice(place.col0, None if place.ncols is None else place.col0 + place.ncols)
    parts = []
    for local, first, count in place.runs(int(full_shape[0])):
        lo, hi = max(local, start), min(local + count, stop)
        if lo < hi:
            r = slice(first + lo - local, first + hi - local)
            parts.append(source[r, cols] if len(full_shape) == 2 else source[r])
    return parts[0] if len(parts) == 1 else torch.cat(parts)


def _local_rows(place: _Placement, full_shape: tuple[int, ...]) -> int:
    return int(full_shape[0]) if place.rows is None else int(place.rows.numel())


# ------------------------------------------------------------------- loading

def _fp32_name_sets(model: Any, params: Iterable[str] | None,
                    buffers: Iterable[str] | None) -> tuple[frozenset, frozenset]:
    defining = sys.modules.get(type(model).__module__)
    if params is None:
        params = getattr(defining, "MINIMAX_H3_FP32_PARAM_NAMES", ())
    if buffers is None:
        buffers = getattr(defining, "MINIMAX_H3_FP32_BUFFER_NAMES", ())
    return frozenset(params), frozenset(buffers)


def load_minimax_h3_dit_weights(model: torch.nn.Module, transformer_root: str | Path, *,
                                maximum_temporary_bytes: int = _STREAM_LOAD_TEMPORARY_BYTES,
                                fp32_param_names: Iterable[str] | None = None,
                                fp32_buffer_names: Iterable[str] | None = None) -> dict[str, Any]:
    """Load a transformer directory into the model's TP-local parameters and
    pending W8 slots, one shard at a time, and return the reference's receipt
    (H3/model/weight_loading.py:154-264)."""
    if not isinstance(model, torch.nn.Module):
        raise TypeError("model must be an nn.Module")
    checkpoint = _Checkpoint(Path(transformer_root))
    safe_open = importlib.import_module("safetensors").safe_open
    state = model.state_dict(keep_vars=True)
    missing = sorted(set(state) - set(checkpoint.location))
    unexpected = sorted(set(checkpoint.location) - set(state))
    if missing or unexpected:
        raise H3NativeWeightError("H3 transformer tensor inventory differs: "
                                  f"missing={missing[:8]}, unexpected={unexpected[:8]}")
    modules = dict(model.named_modules())
    per_shard: dict[Path, list[str]] = {shard: [] for shard in checkpoint.shards}
    for tensor_name, shard in checkpoint.location.items():
        per_shard[shard].append(tensor_name)

    streamed = 0
    totals = {"source": 0, "quantized": 0, "scale": 0, "staging": 0, "bf16": 0}
    with torch.no_grad():
        for shard, names in per_shard.items():
            with safe_open(str(shard), framework="pt", device="cpu") as handle:
                for tensor_name in sorted(names):
                    owner_name, _, leaf = tensor_name.rpartition(".")
                    owner = modules.get(owner_name)
                    if owner is None:
                        raise H3NativeWeightError(f"H3 state owner is absent: {tensor_name}")
                    source = handle.get_slice(tensor_name)
                    full_shape = tuple(int(v) for v in source.get_shape())
                    place = _placement(tensor_name, leaf, full_shape, owner, model)
                    if leaf == "weight" and getattr(owner, "_cutlass_w8a8_stream_load_pending", None) is True:
                        _stream_slot(owner, tensor_name, source, full_shape, place,
                                     maximum_temporary_bytes=maximum_temporary_bytes)
                        streamed += 1
                        totals["source"] += int(owner._cutlass_w8a8_source_weight_bytes)
                        totals["quantized"] += int(owner.weight.numel() * owner.weight.element_size())
                        scale = owner._cutlass_w8a8_weight_scale
                        totals["scale"] += int(scale.numel() * scale.element_size())
                        totals["staging"] = max(totals["staging"],
                                                int(owner._cutlass_w8a8_stream_load_temporary_bytes_limit))
                        continue
                    destination = state[tensor_name]
                    if not full_shape:
                        value = handle.get_tensor(tensor_name)
                    else:
                        value = _read_rows(source, full_shape, place, 0, _local_rows(place, full_shape))
                    if tuple(value.shape) != tuple(destination.shape):
                        raise H3NativeWeightError(f"H3 local tensor shape differs for {tensor_name}: "
                                                  f"{tuple(value.shape)} != {tuple(destination.shape)}")
                    if value.dtype != destination.dtype:
                        raise H3NativeWeightError(f"H3 tensor dtype differs for {tensor_name}: "
                                                  f"{value.dtype} != {destination.dtype}")
                    destination.copy_(value)
                    if leaf == "weight" and value.dtype == torch.bfloat16:
                        totals["bf16"] += 1
    pending = [name for name, module in model.named_modules()
               if getattr(module, "_cutlass_w8a8_stream_load_pending", None) is True]
    if pending:
        raise H3NativeWeightError(f"H3 streamed W8A8 weights were not loaded: {pending[:8]}")
    fp32_params, fp32_buffers = _fp32_name_sets(model, fp32_param_names, fp32_buffer_names)
    for name in sorted(fp32_params):
        if model.get_parameter(name).dtype != torch.float32:
            raise H3NativeWeightError(f"H3 parameter must stay fp32: {name}")
    for name in sorted(fp32_buffers):
        if model.get_buffer(name).dtype != torch.float32:
            raise H3NativeWeightError(f"H3 buffer must stay fp32: {name}")
    receipt = {
        "shard_count": len(checkpoint.shards),
        "tensor_count": len(state),
        "stream_load_policy": getattr(model, "_load_time_w8a8_policy", None),
        "streamed_w8a8_linear_count": streamed,
        "streamed_w8a8_source_weight_bytes": totals["source"],
        "streamed_w8a8_quantized_weight_bytes": totals["quantized"],
        "streamed_w8a8_scale_bytes": totals["scale"],
        "stream_load_bf16_staging_bytes_limit": totals["staging"],
        "bf16_weight_copy_count": totals["bf16"],
    }
    model._native_weight_load_receipt = receipt
    return receipt


def _stream_slot(owner: Any, name: str, source: Any, full_shape: tuple[int, ...], place: _Placement, *,
                 maximum_temporary_bytes: int) -> None:
    """Fill a pending W8 slot from the checkpoint, reading only this rank's rows."""
    if source.get_dtype() not in ("BF16", "bfloat16"):
        raise TypeError(f"{name} streamed CUTLASS W8A8 dtype differs")
    if len(full_shape) != 2:
        raise H3NativeWeightError(f"H3 local tensor shape differs for {name}: {full_shape}")
    rows = _local_rows(place, full_shape)
    cols = int(full_shape[1]) if place.ncols is None else place.ncols
    if (rows, cols) != tuple(owner.weight.shape):
        raise H3NativeWeightError(f"H3 local tensor shape differs for {name}: {(rows, cols)} != "
                                  f"{tuple(owner.weight.shape)}")
    stream_quantize_rows_(owner, rows, cols, lambda start, stop: _read_rows(source, full_shape, place, start, stop),
                          name=name, maximum_temporary_bytes=maximum_temporary_bytes)


__all__ = ["H3NativeWeightError", "load_minimax_h3_dit_weights", "qkv_row_order", "reorder_grouped_qkv_to_qkv"]
