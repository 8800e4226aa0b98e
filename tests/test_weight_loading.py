"""Streamed checkpoint loading (H3/model/weight_loading.py:29-264 and the W8
slots of H3/inference/w8a8.py:66-133) on a toy module tree with the
reference's layer types and names.

CPU: the grouped-QKV reorder against a hand-built layout, the index / shard
resolution errors, the inventory check, and a full bf16 load of rank 1 of a
TP=2 shard (reorder + merged / column / row slicing) from two shards and an
index.  GPU: the same tree with W8 slots on qkv_proj and fc1, streamed by
row-range reads in many small chunks; codes and scales must equal the oracle's
int8 quantizer applied to the reference's reordered, sliced bf16 weight."""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from _util import bits16, to_tiled
import taomate_h3_amd.ops as ops_mod

HEADS, HEAD_DIM, HIDDEN, FFN = 4, 32, 256, 512


def _mods():
    import _toy_layers as toy
    import taomate_h3_amd.weight_loading as wl
    return toy, wl


class _Arch:
    num_attention_heads = HEADS
    attention_head_dim = HEAD_DIM


def _model(tp, device, blocks=2):
    toy, _ = _mods()

    class Attn(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.qkv_proj = toy.ToyMergedColumnLinear(HIDDEN, [HEADS * HEAD_DIM] * 3, bias=False,
                                                      dtype=torch.bfloat16, tp=tp, device=device)
            self.out_proj = toy.ToyRowLinear(HEADS * HEAD_DIM, HIDDEN, bias=True, dtype=torch.bfloat16, tp=tp,
                                             device=device)

    class Mlp(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.fc1 = toy.ToyColumnLinear(HIDDEN, FFN, bias=False, dtype=torch.bfloat16, tp=tp, device=device)
            self.fc2 = toy.ToyRowLinear(FFN, HIDDEN, bias=True, dtype=torch.bfloat16, tp=tp, device=device)

    class Block(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.attn, self.mlp = Attn(), Mlp()
            self.scale_shift_table = torch.nn.Parameter(torch.zeros(6, HIDDEN, dtype=torch.float32, device=device))

    class Model(torch.nn.Module):
        arch = _Arch()

        def __init__(self):
            super().__init__()
            self.blocks = torch.nn.ModuleList(Block() for _ in range(blocks))

    return Model()


def _checkpoint(blocks=2, seed=0):
    """Full (unsharded) tensors; qkv in the grouped per-head layout, plus
    the Q, K, V pieces it was built from."""
    gen = torch.Generator().manual_seed(seed)
    full, pieces = {}, {}
    for b in range(blocks):
        q, k, v = ((torch.randn(HEADS * HEAD_DIM, HIDDEN, generator=gen) * 0.05).to(torch.bfloat16)
                   for _ in range(3))
        grouped = torch.cat([torch.cat([t[h * HEAD_DIM:(h + 1) * HEAD_DIM] for t in (q, k, v)])
                             for h in range(HEADS)])
        full[f"blocks.{b}.attn.qkv_proj.weight"] = grouped
        pieces[b] = (q, k, v)
        full[f"blocks.{b}.attn.out_proj.weight"] = (torch.randn(HIDDEN, HEADS * HEAD_DIM, generator=gen)
                                                    * 0.05).to(torch.bfloat16)
        full[f"blocks.{b}.attn.out_proj.bias"] = torch.randn(HIDDEN, generator=gen).to(torch.bfloat16)
        full[f"blocks.{b}.mlp.fc1.weight"] = (torch.randn(FFN, HIDDEN, generator=gen) * 0.05).to(torch.bfloat16)
        full[f"blocks.{b}.mlp.fc2.weight"] = (torch.randn(HIDDEN, FFN, generator=gen) * 0.05).to(torch.bfloat16)
        full[f"blocks.{b}.mlp.fc2.bias"] = torch.randn(HIDDEN, generator=gen).to(torch.bfloat16)
        full[f"blocks.{b}.scale_shift_table"] = torch.randn(6, HIDDEN, generator=gen)
    return full, pieces


def _write(root, full, shards=2, index=True):
    names = sorted(full)
    weight_map = {}
    for s in range(shards):
        part = {n: full[n].contiguous() for n in names[s::shards]}
        fname = f"diffusion_pytorch_model-{s + 1:05d}-of-{shards:05d}.safetensors"
        save_file(part, str(root / fname))
        weight_map.update({n: fname for n in part})
    if index:
        (root / "diffusion_pytorch_model.safetensors.index.json").write_text(json.dumps({"weight_map": weight_map}))


def _expected_local(full, pieces, rank, tp):
    """The reference's local tensors, built from the pieces (not from the
    loader's row map)."""
    out = {}
    for name, value in full.items():
        b = int(name.split(".")[1])
        if name.endswith("qkv_proj.weight"):
            n = HEADS * HEAD_DIM // tp
            out[name] = torch.cat([t[rank * n:(rank + 1) * n] for t in pieces[b]])
        elif name.endswith("fc1.weight"):
            n = FFN // tp
            out[name] = value[rank * n:(rank + 1) * n]
        elif name.endswith(("out_proj.weight", "fc2.weight")):
            k = value.shape[1] // tp
            out[name] = value[:, rank * k:(rank + 1) * k]
        else:
            out[name] = value
    return out


def test_reorder_grouped_qkv_matches_hand_layout():
    _, wl = _mods()
    rows = torch.arange(8).view(8, 1)  # groups of (q, q, k, v): q00 q01 k0 v0 q10 q11 k1 v1
    out = wl.reorder_grouped_qkv_to_qkv(rows, num_query_groups=2, heads_per_group=2, head_dim=1)
    assert out.view(-1).tolist() == [0, 1, 4, 5, 2, 6, 3, 7]
    two = torch.arange(24).view(12, 2)  # head_dim 2, one query head per group
    out = wl.reorder_grouped_qkv_to_qkv(two, num_query_groups=2, heads_per_group=1, head_dim=2)
    assert out[:, 0].tolist() == [0, 2, 12, 14, 4, 6, 16, 18, 8, 10, 20, 22]
    with pytest.raises(wl.H3NativeWeightError, match="grouped"):
        wl.reorder_grouped_qkv_to_qkv(torch.zeros(7, 2), num_query_groups=2, heads_per_group=1, head_dim=1)


@pytest.mark.parametrize("index", [True, False])
def test_bf16_load_of_a_tp_rank(tmp_path, index):
    _, wl = _mods()
    full, pieces = _checkpoint()
    _write(tmp_path, full, index=index)
    model = _model((2, 1), "cpu")
    receipt = wl.load_minimax_h3_dit_weights(model, tmp_path)
    expect = _expected_local(full, pieces, rank=1, tp=2)
    state = model.state_dict()
    for name, value in expect.items():
        assert torch.equal(state[name], value), name
    assert receipt["shard_count"] == 2 and receipt["tensor_count"] == len(full)
    assert receipt["streamed_w8a8_linear_count"] == 0 and receipt["bf16_weight_copy_count"] == 8
    assert model._native_weight_load_receipt is receipt


def test_fp32_parameters_and_buffers_are_checked(tmp_path):
    """H3/model/weight_loading.py:246-251: named parameters and buffers must
    still be fp32 after the load; the name sets default to the constants of
    the module that defines the model class, or are passed in."""
    _, wl = _mods()
    full, _ = _checkpoint(blocks=1)
    _write(tmp_path, full, shards=1)
    model = _model((1, 0), "cpu", blocks=1)
    model.register_buffer("inv_freq", torch.ones(4, dtype=torch.float32), persistent=False)
    wl.load_minimax_h3_dit_weights(model, tmp_path, fp32_param_names={"blocks.0.scale_shift_table"},
                                   fp32_buffer_names={"inv_freq"})
    with pytest.raises(wl.H3NativeWeightError, match="parameter must stay fp32: blocks.0.mlp.fc1.weight"):
        wl.load_minimax_h3_dit_weights(model, tmp_path, fp32_param_names={"blocks.0.mlp.fc1.weight"})
    model.inv_freq = model.inv_freq.to(torch.bfloat16)
    with pytest.raises(wl.H3NativeWeightError, match="buffer must stay fp32: inv_freq"):
        wl.load_minimax_h3_dit_weights(model, tmp_path, fp32_buffer_names={"inv_freq"})
    # default: the name sets of the module defining the model class
    import sys

    this = sys.modules[type(model).__module__]
    this.MINIMAX_H3_FP32_BUFFER_NAMES = frozenset({"inv_freq"})
    try:
        with pytest.raises(wl.H3NativeWeightError, match="buffer must stay fp32"):
            wl.load_minimax_h3_dit_weights(model, tmp_path)
    finally:
        del this.MINIMAX_H3_FP32_BUFFER_NAMES


def test_index_and_inventory_errors(tmp_path):
    _, wl = _mods()
    full, _ = _checkpoint(blocks=1)
    model = _model((1, 0), "cpu", blocks=1)
    with pytest.raises(wl.H3NativeWeightError, match="cannot resolve"):
        wl.load_minimax_h3_dit_weights(model, tmp_path / "absent")
    (tmp_path / "file").write_text("")
    with pytest.raises(wl.H3NativeWeightError, match="must be a directory"):
        wl.load_minimax_h3_dit_weights(model, tmp_path / "file")
    (tmp_path / "file").unlink()
    with pytest.raises(wl.H3NativeWeightError, match="safetensors are absent"):
        wl.load_minimax_h3_dit_weights(model, tmp_path)
    _write(tmp_path, full, shards=1, index=True)
    (tmp_path / "model.safetensors.index.json").write_text("{}")
    with pytest.raises(wl.H3NativeWeightError, match="multiple"):
        wl.load_minimax_h3_dit_weights(model, tmp_path)
    (tmp_path / "model.safetensors.index.json").unlink()
    index = tmp_path / "diffusion_pytorch_model.safetensors.index.json"
    index.write_text(json.dumps({"weight_map": {"a": "../x.safetensors"}}))
    with pytest.raises(wl.H3NativeWeightError, match="escapes"):
        wl.load_minimax_h3_dit_weights(model, tmp_path)
    index.write_text(json.dumps({"weight_map": {}}))
    with pytest.raises(wl.H3NativeWeightError, match="weight_map is absent"):
        wl.load_minimax_h3_dit_weights(model, tmp_path)
    index.write_text(json.dumps({"weight_map": {n: "diffusion_pytorch_model-00001-of-00001.safetensors"
                                                for n in list(full)[1:]}}))
    with pytest.raises(wl.H3NativeWeightError, match="inventory differs"):
        wl.load_minimax_h3_dit_weights(model, tmp_path)
    index.unlink()
    save_file({"blocks.0.mlp.fc2.bias": full["blocks.0.mlp.fc2.bias"]}, str(tmp_path / "dup.safetensors"))
    with pytest.raises(wl.H3NativeWeightError, match="duplicate"):
        wl.load_minimax_h3_dit_weights(model, tmp_path)


@pytest.mark.gpu
def test_streamed_w8a8_slots_match_the_oracle(tmp_path, oracle, device):
    """W8 slots on qkv_proj (grouped reorder + merged TP slice) and fc1
    (column slice), rank 1 of TP=2, 4 KiB of staging: codes and scales equal
    the oracle's quantizer of the reference's local weights."""
    _, wl = _mods()
    from taomate_h3_amd.inference import w8a8

    full, pieces = _checkpoint()
    _write(tmp_path, full)
    model = _model((2, 1), device)
    slots = ["blocks.1.attn.qkv_proj", "blocks.0.mlp.fc1", "blocks.1.mlp.fc1"]
    for name in slots:
        w8a8.prepare_cutlass_w8a8_stream_load_slot_(model.get_submodule(name), name=name)
    print("streamed load: 3 W8 slots, tp rank 1 of 2", flush=True)
    receipt = wl.load_minimax_h3_dit_weights(model, tmp_path, maximum_temporary_bytes=4096)
    torch.cuda.synchronize()
    assert receipt["streamed_w8a8_linear_count"] == 3
    assert receipt["stream_load_bf16_staging_bytes_limit"] == 4096
    expect = _expected_local(full, pieces, rank=1, tp=2)
    for name in slots:
        module = model.get_submodule(name)
        rq, rs = oracle.quant_rows(bits16(expect[name + ".weight"]), "int8", "div")
        assert ops_mod.is_tiled(module.weight)
        np.testing.assert_array_equal(module.weight.detach().view(torch.uint8).cpu().numpy(),
                                      to_tiled(rq.view(np.uint8)))
        np.testing.assert_array_equal(module._cutlass_w8a8_weight_scale.cpu().numpy().ravel(), rs)
        assert module._cutlass_w8a8_stream_loaded and not module._cutlass_w8a8_stream_load_pending
    # the bf16 tensors of the same checkpoint land as in the CPU load
    state = model.state_dict()
    for name in ("blocks.0.attn.qkv_proj.weight", "blocks.1.attn.out_proj.weight", "blocks.0.mlp.fc2.weight"):
        assert torch.equal(state[name].cpu(), expect[name]), name
    # the loaded int8 linear runs: rank 1's fc1 output columns
    x = (torch.randn(32, HIDDEN, generator=torch.Generator().manual_seed(3))).to(torch.bfloat16)
    out = model.get_submodule("blocks.0.mlp.fc1")(x.to(device))
    torch.cuda.synchronize()
    assert tuple(out.shape) == (32, FFN // 2)
