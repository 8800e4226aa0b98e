"""Host-side behaviour of the reference-interface mirror (CPU only).

Policy resolution (H3/inference/w8a8.py:29-54, FL/inference/fp8.py:23-93),
the stream-load slot protocol (H3/inference/w8a8.py:66-133), and the
errors raised before any launch, with the reference's messages."""

from __future__ import annotations

import importlib

import pytest
import torch

w8a8 = importlib.import_module("taomate_h3_amd.inference.w8a8")
fp8 = importlib.import_module("taomate_h3_amd.inference.fp8")
linear = importlib.import_module("taomate_h3_amd.distributed.linear")
ops = importlib.import_module("taomate_h3_amd.ops")

NAMES = [f"blocks.{b}.{p}" for b in range(50) for p in ("attn.qkv_proj", "attn.out_proj", "mlp.fc1", "mlp.fc2")]


def test_int8_policy_selects_interior_qkv_and_fc1():
    sel = w8a8.resolve_h3_cutlass_w8a8_policy(NAMES, policy="interior_fc1_qkv_v1")
    q = sel["quantized_linear_names"]
    assert len(q) == 90  # blocks 2..46, qkv + fc1: 90 linears
    assert all(n.endswith((".attn.qkv_proj", ".mlp.fc1")) for n in q)
    assert {int(n.split(".")[1]) for n in q} == set(range(2, 47))
    assert sel["bf16_boundary_block_indices"] == [0, 1, 47, 48, 49]
    # out_proj is not a candidate at all; fc2 and boundary qkv/fc1 stay bf16
    assert len(sel["bf16_protected_linear_names"]) == 50 + 10
    assert not any(n.endswith("out_proj") for n in sel["bf16_protected_linear_names"])


def test_int8_policy_errors():
    with pytest.raises(ValueError, match="unsupported H3 W8A8 policy"):
        w8a8.resolve_h3_cutlass_w8a8_policy(NAMES, policy="bogus")
    with pytest.raises(RuntimeError, match="found no DiT projections"):
        w8a8.resolve_h3_cutlass_w8a8_policy(["proj_out"], policy="interior_fc1_qkv_v1")


@pytest.mark.parametrize("policy,qkv_blocks,fc1", [
    ("quality_first_residual_v1", list(range(2, 47)), 45),
    ("interior_fc1_only_v1", [], 45),
    ("interior_fc1_mid18_qkv_v1", list(range(16, 34)), 45),
])
def test_fp8_policies(policy, qkv_blocks, fc1):
    sel = fp8.resolve_h3_dynamic_fp8_policy(NAMES, policy=policy)
    q = sel["quantized_linear_names"]
    assert sum(n.endswith("mlp.fc1") for n in q) == fc1
    assert sel["quantized_qkv_block_indices"] == qkv_blocks
    assert not any(n.endswith(("out_proj", "fc2")) for n in q)
    assert sel["bf16_boundary_block_indices"] == [0, 1, 47, 48, 49]


def test_fp8_receipt_policy_rules_and_projection_sets():
    """The receipt fields FL/inference/fp8.py:288-372 derives from the policy,
    with the reference's literal strings."""
    boundary = [0, 1, 47, 48, 49]
    fc1_only = fp8._policy_rules("interior_fc1_only_v1",
                                 fp8.resolve_h3_dynamic_fp8_policy(NAMES, policy="interior_fc1_only_v1"))
    assert fc1_only == {
        "quantized_projection_suffixes": ["mlp.fc1"],
        "bf16_projection_suffixes": ["attn.qkv_proj", "attn.out_proj", "mlp.fc2"],
        "bf16_boundary_block_indices": boundary,
        "quantized_qkv_block_indices": [],
        "bf16_qkv_block_indices": list(range(50)),
        "reason": "protect attention, residual-write projections, and both representation boundaries "
                  "(first two and last three blocks)",
    }
    mid = fp8._policy_rules("interior_fc1_mid18_qkv_v1",
                            fp8.resolve_h3_dynamic_fp8_policy(NAMES, policy="interior_fc1_mid18_qkv_v1"))
    assert mid["quantized_projection_suffixes"] == ["attn.qkv_proj", "mlp.fc1"]
    assert mid["bf16_projection_suffixes"] == ["attn.out_proj", "mlp.fc2"]
    assert mid["quantized_qkv_block_indices"] == list(range(16, 34))
    assert mid["bf16_qkv_block_indices"] == [b for b in range(50) if not 16 <= b <= 33]
    assert mid["reason"] == ("protect QKV outside blocks 16 through 33, all residual-write projections, "
                             "and both representation boundaries")
    qf = fp8._policy_rules("quality_first_residual_v1",
                           fp8.resolve_h3_dynamic_fp8_policy(NAMES, policy="quality_first_residual_v1"))
    assert qf["reason"] == ("protect residual-write projections and both representation boundaries "
                            "(first two and last three blocks)")
    assert qf["bf16_qkv_block_indices"] == boundary
    assert fp8._policy_rules(None, fp8.resolve_h3_dynamic_fp8_policy(NAMES, policy=None)) is None
    assert [fp8._projection_set(p, False) for p in (None, "interior_fc1_only_v1", "interior_fc1_mid18_qkv_v1",
                                                    "quality_first_residual_v1")] == [
        "attention_and_mlp", "mlp_input_interior_blocks", "mlp_input_interior_and_mid18_qkv_blocks",
        "qkv_and_mlp_input_interior_blocks"]
    assert fp8._projection_set(None, True) == "mlp_only"


def test_fp8_policy_none_and_errors():
    assert fp8.resolve_h3_dynamic_fp8_policy(NAMES, policy=None)["quantized_linear_names"] == NAMES
    with pytest.raises(ValueError, match="unsupported H3 dynamic FP8 policy"):
        fp8.resolve_h3_dynamic_fp8_policy(NAMES, policy="x")
    with pytest.raises(ValueError, match="requires eligible linear names"):
        fp8.resolve_h3_dynamic_fp8_policy([], policy=None)


class _Proj(torch.nn.Module):
    def __init__(self, n=8, k=16, bias=False, device="cpu"):
        super().__init__()
        self.weight = torch.nn.Parameter(torch.empty(n, k, dtype=torch.bfloat16, device=device))
        self.bias = torch.nn.Parameter(torch.zeros(n, dtype=torch.bfloat16)) if bias else None


def test_stream_load_slot_replaces_weight_with_int8_storage():
    m = _Proj(device="meta")
    w8a8.prepare_cutlass_w8a8_stream_load_slot_(m, name="blocks.3.mlp.fc1")
    assert m.weight.dtype == torch.int8 and m.weight.requires_grad is False
    assert tuple(m._cutlass_w8a8_weight_scale.shape) == (8, 1)
    assert m._cutlass_w8a8_weight_scale.dtype == torch.float32
    assert "_cutlass_w8a8_weight_scale" not in m.state_dict()
    assert m._cutlass_w8a8_stream_load_pending is True and m._cutlass_w8a8_stream_loaded is False
    assert m._cutlass_w8a8_source_weight_bytes == 8 * 16 * 2


def test_stream_load_slot_errors():
    m = _Proj()
    m.weight.data = m.weight.data.float()
    with pytest.raises(TypeError, match="expected an uninitialized BF16 weight"):
        w8a8.prepare_cutlass_w8a8_stream_load_slot_(m, name="x")
    m = _Proj()
    m.weight.requires_grad_(False)
    with pytest.raises(RuntimeError, match="already frozen"):
        w8a8.prepare_cutlass_w8a8_stream_load_slot_(m, name="x")
    with pytest.raises(RuntimeError, match="bias-free H3 projection"):
        w8a8.prepare_cutlass_w8a8_stream_load_slot_(_Proj(bias=True), name="x")


def test_stream_load_errors_before_any_launch():
    m = _Proj()
    src = torch.zeros(8, 16, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="no pending CUTLASS W8A8 stream load"):
        w8a8.load_cutlass_w8a8_stream_weight_(m, src, name="x")
    w8a8.prepare_cutlass_w8a8_stream_load_slot_(m, name="x")
    with pytest.raises(TypeError, match="dtype differs"):
        w8a8.load_cutlass_w8a8_stream_weight_(m, src.float(), name="x")
    with pytest.raises(ValueError, match="shape differs"):
        w8a8.load_cutlass_w8a8_stream_weight_(m, src[:4], name="x")
    with pytest.raises(ValueError, match="must be positive"):
        w8a8.load_cutlass_w8a8_stream_weight_(m, src, name="x", maximum_temporary_bytes=0)


def test_linear_bias_rejected_like_reference():
    with pytest.raises(RuntimeError, match="bias-free linears only"):
        w8a8.cutlass_w8a8_linear(torch.zeros(2, 16), torch.zeros(8, 16, dtype=torch.int8), torch.ones(8, 1),
                                 bias=torch.zeros(8), workspace=None, weight_t=None, weight_scale_t=None)


def test_fl_dispatch_rejects_two_quantizers():
    with pytest.raises(RuntimeError, match="cannot combine CUTLASS W8A8"):
        linear._linear(torch.zeros(2, 16), torch.zeros(8, 16), None, torch.ones(()), None, torch.ones(8, 1))


def test_bf16_module_linear_is_plain_linear():
    from _toy_layers import ToyColumnLinear

    m = ToyColumnLinear(16, 8, bias=True, dtype=torch.float32)
    torch.nn.init.normal_(m.weight)
    torch.nn.init.normal_(m.bias)
    x = torch.randn(3, 16)
    assert torch.allclose(m(x), torch.nn.functional.linear(x, m.weight, m.bias))


def test_lora_wrapper_switch_and_cross_rank_guard():
    """adapter_enabled off returns the base output alone (FL/inference/lora_checkpoint.py:452-489);
    a row-parallel base split over ranks raises instead of returning a partial."""
    from _toy_layers import ToyColumnLinear, ToyRowLinear
    from taomate_h3_amd.inference import lora

    base = ToyColumnLinear(16, 8, bias=False, dtype=torch.float32)
    torch.nn.init.normal_(base.weight)
    a, b = torch.randn(4, 16), torch.randn(8, 4)
    wrapped = lora.H3InferenceParallelLinearLoRA(base, kind="column", a=a, b=b, scale=0.5)
    x = torch.randn(3, 16)
    assert torch.allclose(wrapped(x), base(x) + (x @ a.t() @ b.t()) * 0.5, atol=1e-5)
    wrapped.adapter_enabled = False
    assert torch.equal(wrapped(x), base(x))
    row = ToyRowLinear(16, 8, bias=False, dtype=torch.float32, tp=(2, 1))
    torch.nn.init.normal_(row.weight)
    wrapped_row = lora.H3InferenceParallelLinearLoRA(row, kind="row", a=torch.randn(4, 8), b=b, scale=1.0)
    with pytest.raises(NotImplementedError, match="across tensor-parallel ranks"):
        wrapped_row(torch.randn(3, 8))


def test_lora_merge_and_base_model_bypass():
    """FL's merge (fp32 delta, one rounding to the base dtype) and the
    base-model context that switches adapters off and restores them."""
    from _toy_layers import ToyColumnLinear
    from taomate_h3_amd.inference import lora

    root = torch.nn.Module()
    root.proj = ToyColumnLinear(16, 8, bias=False, dtype=torch.bfloat16)
    torch.nn.init.normal_(root.proj.weight)
    w0 = root.proj.weight.detach().clone()
    a = torch.randn(4, 16).to(torch.bfloat16)
    b = torch.randn(8, 4).to(torch.bfloat16)
    root.proj = lora.H3InferenceParallelLinearLoRA(root.proj, kind="column", a=a, b=b, scale=0.25)
    with lora.h3_base_model_inference(root):
        assert root.proj.adapter_enabled is False
    assert root.proj.adapter_enabled is True
    receipt = lora.merge_h3_lora_weights_(root)
    expect = (w0.float() + (b.float() @ a.float()) * 0.25).to(torch.bfloat16)
    assert torch.equal(root.proj.base.weight, expect)
    assert receipt["target_count"] == 1 and receipt["reversible"] is False
    assert root.proj.adapter_enabled is False and not hasattr(root.proj, "lora_a")
    with pytest.raises(lora.H3LoRACheckpointError, match="already merged"):
        with lora.h3_base_model_inference(root):
            pass


def _lora_toy_model(tp=(1, 0)):
    from _toy_layers import ToyColumnLinear, ToyRowLinear

    root = torch.nn.Module()
    root.blocks = torch.nn.ModuleList()
    for _ in range(2):
        block = torch.nn.Module()
        block.attn = torch.nn.Module()
        block.attn.qkv_proj = ToyColumnLinear(32, 96, bias=False, dtype=torch.bfloat16, tp=tp)
        block.attn.out_proj = ToyRowLinear(32, 32, bias=True, dtype=torch.bfloat16, tp=tp)
        root.blocks.append(block)
    return root


@pytest.mark.parametrize("marker", ["_taomate_h3_inference_lora", "_digitalhuman_h3_inference_lora"])
def test_fuse_lora_wrappers_swaps_reference_wrappers(marker):
    """fuse_h3_lora_wrappers_ replaces the wrappers the reference's
    apply_h3_lora_checkpoint installs (H3/inference/lora_checkpoint.py:172-246,
    FL :440-553) in their parents, keeping base, kind, scale, the same buffer
    tensors, the row-reduce and adapter switches and the package's marker."""
    from _toy_layers import install_reference_lora
    from taomate_h3_amd.inference import lora

    root = _lora_toy_model()
    names = ["blocks.0.attn.qkv_proj", "blocks.0.attn.out_proj", "blocks.1.attn.qkv_proj"]
    installed = install_reference_lora(root, names, rank=8, scale=0.5, seed=3, marker=marker)
    installed["blocks.0.attn.out_proj"].fused_row_reduce_enabled = True
    if marker == "_digitalhuman_h3_inference_lora":
        installed["blocks.1.attn.qkv_proj"].adapter_enabled = False
    receipt = lora.fuse_h3_lora_wrappers_(root)
    assert receipt["target_count"] == 3 and receipt["replaced_count"] == 3
    assert receipt["already_fused_wrapper_count"] == 0 and receipt["kept_reference_wrapper_names"] == []
    assert receipt["fused_epilogue_ready_count"] == 0  # bf16 toy bases, not W8A8
    for name, old in installed.items():
        new = root.get_submodule(name)
        assert isinstance(new, lora.H3InferenceParallelLinearLoRA)
        assert new.base is old.base and new.kind == old.kind and new.scale == old.scale
        assert new.lora_a is old.lora_a and new.lora_b is old.lora_b
        assert getattr(new, marker) is True and new._taomate_h3_inference_lora is True
        assert new.fused_row_reduce_enabled == old.fused_row_reduce_enabled
        assert new.adapter_enabled == getattr(old, "adapter_enabled", True)
        assert not new.training
    # the reference's later passes still find the adapters; a second swap replaces nothing
    assert lora.materialize_h3_lora_bf16_buffers_(root)["target_count"] == 3
    again = lora.fuse_h3_lora_wrappers_(root)
    assert again["replaced_count"] == 0 and again["already_fused_wrapper_count"] == 3


def test_fuse_lora_wrappers_validates_before_replacing():
    """A wrapper whose buffers do not fit its base fails the whole call before
    any wrapper is replaced; a model without adapters raises; a row-parallel
    wrapper over several ranks stays the reference's (it needs the cross-rank
    reduce)."""
    from _toy_layers import ToyReferenceLoRAWrapper, install_reference_lora
    from taomate_h3_amd.inference import lora

    with pytest.raises(lora.H3LoRACheckpointError, match="requires a loaded inference LoRA adapter"):
        lora.fuse_h3_lora_wrappers_(_lora_toy_model())
    root = _lora_toy_model()
    install_reference_lora(root, ["blocks.0.attn.qkv_proj"], rank=8, scale=1.0, seed=4)
    bad_base = root.blocks[1].attn.qkv_proj
    root.blocks[1].attn.qkv_proj = ToyReferenceLoRAWrapper(bad_base, kind="column", a=torch.zeros(8, 31),
                                                           b=torch.zeros(96, 8), scale=1.0)
    with pytest.raises(lora.H3LoRACheckpointError, match="local shape differs: blocks.1.attn.qkv_proj"):
        lora.fuse_h3_lora_wrappers_(root)
    assert not isinstance(root.blocks[0].attn.qkv_proj, lora.H3InferenceParallelLinearLoRA)
    split = _lora_toy_model(tp=(2, 0))
    install_reference_lora(split, ["blocks.0.attn.qkv_proj", "blocks.0.attn.out_proj"], rank=8, scale=1.0, seed=5)
    receipt = lora.fuse_h3_lora_wrappers_(split)
    assert receipt["replaced_count"] == 1 and receipt["kept_reference_wrapper_names"] == ["blocks.0.attn.out_proj"]
    assert isinstance(split.blocks[0].attn.qkv_proj, lora.H3InferenceParallelLinearLoRA)
    assert not isinstance(split.blocks[0].attn.out_proj, lora.H3InferenceParallelLinearLoRA)


def test_ops_reject_host_tensors_before_launch():
    x = torch.zeros(4, 16, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.quant_rows(x, ops.FMT_E4M3FN)
    a = torch.zeros(4, 16, dtype=torch.int8)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.scaled_mm(a, a, torch.ones(4), torch.ones(4))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.lora_down(x, x)


def test_int8_stream_chunking_matches_whole_matrix_on_host_formula():
    """The reference's claim (H3/inference/w8a8.py:105-110): row chunks with
    per-row scales equal whole-matrix quantization -- checked on the oracle."""
    from oracle import oracle as O
    from _util import bits16, weights

    w = weights(37, 96, seed=3)
    whole_q, whole_s = O.quant_rows(bits16(w), "int8", "div")
    parts = [O.quant_rows(bits16(w[i:i + 5]), "int8", "div") for i in range(0, 37, 5)]
    import numpy as np

    assert np.array_equal(np.concatenate([p[0] for p in parts]), whole_q)
    assert np.array_equal(np.concatenate([p[1] for p in parts]), whole_s)


def test_fused_norm_mirrors_check_indices_and_devices():
    """fused_rms_norm_modulate keeps the reference's index check
    (H3/inference/fused_kernels.py:711-713) and, like every op here, refuses
    host tensors before any launch."""
    from taomate_h3_amd.inference import fused_kernels as fk

    x = torch.zeros(2, 3, 16, dtype=torch.bfloat16)
    w = torch.ones(16, dtype=torch.bfloat16)
    tab = torch.zeros(2, 16, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="SOL RMSNorm/AdaLN indices do not cover every row"):
        fk.fused_rms_norm_modulate(x, w, tab, tab, torch.zeros(5, dtype=torch.int64), 1e-6)
    with pytest.raises(ValueError, match="SOL residual/AdaLN indices do not cover every row"):
        fk.fused_residual_gate_rms_norm_modulate(x, x, tab, w, tab, tab, torch.zeros(7, dtype=torch.int64), 1e-6)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        fk.fused_rms_norm_modulate(x, w, tab, tab, torch.zeros(6, dtype=torch.int64), 1e-6)
    with pytest.raises(TypeError, match="bfloat16"):
        fk.fused_rms_norm_modulate_w8a8(x.float(), w, tab, tab, torch.zeros(6, dtype=torch.int64), 1e-6)
    qa = fk.QuantizedActivations(torch.zeros(6, 16, dtype=torch.int8), torch.ones(6, 1), (2, 3, 16))
    with pytest.raises(TypeError, match="keep_dense=True"):
        fk.as_dense(qa)


def test_tiled_mark_lives_with_the_storage():
    """The tiled mark belongs to the storage: a view that outlives the marked
    parameter still reads as tiled; the entry goes when the last view goes;
    a copy is not tiled."""
    import gc

    param = torch.nn.Parameter(torch.zeros(32, 256, dtype=torch.int8), requires_grad=False)
    ops.mark_tiled(param)
    view = param.t()
    key = ops._storage_key(param)
    assert ops.is_tiled(view) and ops.is_tiled(param.data) and ops.is_tiled(param.detach()[:16])
    assert not ops.is_tiled(param.detach().clone())
    del param
    gc.collect()
    assert ops.is_tiled(view) and key in ops._TILED_STORAGES
    del view
    gc.collect()
    assert key not in ops._TILED_STORAGES
    with pytest.raises(ValueError, match="whole storage"):
        ops.mark_tiled(torch.zeros(32, 256, dtype=torch.int8)[:16])


def test_tiled_weight_survives_deepcopy_of_its_module():
    """copy.deepcopy of a module whose weight this package stored tiled gives
    new, unmarked storage; the module records the layout, and the dispatch
    re-marks the copy (ops.module_weight_tiled), so the copy computes what the
    original does.  The weight_t view copied beside it resolves to the same storage."""
    import copy

    m = torch.nn.Module()
    m.weight = torch.nn.Parameter(torch.zeros(32, 256, dtype=torch.int8), requires_grad=False)
    ops.mark_module_weight_tiled(m)
    m._cutlass_w8a8_weight_t = m.weight.t()
    twin = copy.deepcopy(m)
    assert twin.weight.untyped_storage().data_ptr() != m.weight.untyped_storage().data_ptr()
    assert not ops.is_tiled(twin.weight) and not ops.is_tiled(twin._cutlass_w8a8_weight_t)
    assert ops.module_weight_tiled(twin)
    assert ops.is_tiled(twin.weight) and ops.is_tiled(twin._cutlass_w8a8_weight_t)
    assert ops.module_weight_tiled(m)
    plain = torch.nn.Module()
    plain.weight = torch.nn.Parameter(torch.zeros(32, 256, dtype=torch.int8), requires_grad=False)
    assert not ops.module_weight_tiled(plain)
    twin.weight = torch.nn.Parameter(torch.zeros(30, 256, dtype=torch.int8), requires_grad=False)
    with pytest.raises(ValueError, match="not a tiled code matrix"):
        ops.module_weight_tiled(twin)
