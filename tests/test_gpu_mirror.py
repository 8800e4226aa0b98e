"""The reference-interface mirror on the GPU, checked against the oracle.

Covers the int8 W8A8 module path (H3/inference/w8a8.py:98-220), the FP8
quantizers of FL/inference/fused_kernels.py:771-820, the FL linear dispatch
(FL/distributed/linear.py:50-128 with H3/distributed/linear.py:15-33) and the
fused LoRA wrapper (H3/inference/lora_checkpoint.py:172-205)."""

from __future__ import annotations

import importlib

import numpy as np
import pytest
import torch

from _util import activations, bits8, bits16, to_tiled, weights
from test_gpu_gemm import _assert_fp8_close
import taomate_h3_amd.ops as ops_mod

pytestmark = pytest.mark.gpu

PKG = "taomate_h3_amd"


def _mod(name):
    return importlib.import_module(f"{PKG}.{name}")


def _int8_reference(oracle, x, w):
    rqa, rsa = oracle.quant_rows(bits16(x), "int8", "rcp")
    rqw, rsw = oracle.quant_rows(bits16(w), "int8", "div")
    return oracle.epilogue(oracle.gemm_i8_i32_fast(rqa, rqw), rsa, rsw)


class _Block(torch.nn.Module):
    def __init__(self, d, hidden, device):
        super().__init__()
        from _toy_layers import ToyColumnLinear, ToyRowLinear

        self.attn = torch.nn.Module()
        self.mlp = torch.nn.Module()
        kw = dict(dtype=torch.bfloat16, device=device)
        self.attn.qkv_proj = ToyColumnLinear(d, 3 * d, bias=False, **kw)
        self.attn.out_proj = ToyRowLinear(d, d, bias=True, **kw)
        self.mlp.fc1 = ToyColumnLinear(d, hidden, bias=False, **kw)
        self.mlp.fc2 = ToyRowLinear(hidden, d, bias=True, **kw)


class _Transformer(torch.nn.Module):
    def __init__(self, blocks=7, d=256, hidden=512, device="cuda"):
        super().__init__()
        self.blocks = torch.nn.ModuleList(_Block(d, hidden, device) for _ in range(blocks))
        gen = torch.Generator().manual_seed(4)
        for p in self.parameters():
            p.data.copy_((torch.randn(p.shape, generator=gen) * 0.03).to(torch.bfloat16))


def test_quantize_weight_matches_reference_formula(oracle, device):
    w8a8 = _mod("inference.w8a8")
    w = weights(96, 640, seed=7)
    q, s = w8a8._quantize_weight(w.to(device))
    rq, rs = oracle.quant_rows(bits16(w), "int8", "div")
    np.testing.assert_array_equal(bits8(q).view(np.int8), rq)
    np.testing.assert_array_equal(s.cpu().numpy().ravel(), rs)


@pytest.mark.parametrize("rows,k,limit", [(300, 512, 1024 * 1024), (300, 512, 512 * 2 * 7), (5, 256, 1),
                                         (320, 512, 512 * 2 * 7), (64, 1024, 1)])
def test_stream_load_chunks_equal_whole_matrix(oracle, device, rows, k, limit):
    """Bounded row chunks (w8a8.py:98-133) give the whole-matrix codes and
    scales; aligned shapes are written straight into the tiled layout."""
    w8a8 = _mod("inference.w8a8")
    m = torch.nn.Module()
    m.weight = torch.nn.Parameter(torch.empty(rows, k, dtype=torch.bfloat16, device=device))
    m.bias = None
    w8a8.prepare_cutlass_w8a8_stream_load_slot_(m, name="blocks.2.mlp.fc1")
    src = weights(rows, k, seed=rows)
    w8a8.load_cutlass_w8a8_stream_weight_(m, src, name="blocks.2.mlp.fc1", maximum_temporary_bytes=limit)
    torch.cuda.synchronize()
    rq, rs = oracle.quant_rows(bits16(src), "int8", "div")
    tiled = rows % 16 == 0 and k % 128 == 0
    assert ops_mod.is_tiled(m.weight) == tiled
    expect = to_tiled(rq.view(np.uint8)) if tiled else rq.view(np.uint8)
    np.testing.assert_array_equal(bits8(m.weight), expect)
    np.testing.assert_array_equal(m._cutlass_w8a8_weight_scale.cpu().numpy().ravel(), rs)
    assert m._cutlass_w8a8_stream_loaded is True and m._cutlass_w8a8_stream_load_pending is False


@pytest.mark.parametrize("shape", [(2, 150, 512), (1, 1, 512), (640, 512)])
def test_cutlass_w8a8_linear_bit_exact(oracle, device, shape):
    w8a8 = _mod("inference.w8a8")
    k, n = shape[-1], 384
    x = activations(int(np.prod(shape[:-1])), k, seed=3, outlier_channels=4).reshape(shape)
    w = weights(n, k, seed=5)
    qw, sw = w8a8._quantize_weight(w.to(device))
    out = w8a8.cutlass_w8a8_linear(x.to(device), qw, sw, bias=None, workspace=None, weight_t=None,
                                   weight_scale_t=None)
    torch.cuda.synchronize()
    assert tuple(out.shape) == (*shape[:-1], n) and out.dtype == torch.bfloat16
    ref = _int8_reference(oracle, x.reshape(-1, k), w)
    np.testing.assert_array_equal(bits16(out).reshape(-1, n), ref)


def test_workspace_path_equal_and_aliased(oracle, device):
    """The workspace path returns the same bits as the allocating path, and
    same-width outputs on one stream share storage (w8a8.py:136-187)."""
    w8a8 = _mod("inference.w8a8")
    k, n = 512, 768
    w = weights(n, k, seed=8)
    qw, sw = w8a8._quantize_weight(w.to(device))
    ws = w8a8.CutlassW8A8Workspace()
    x1 = activations(200, k, seed=1, outlier_channels=3)
    x2 = activations(120, k, seed=2, outlier_channels=3)
    o1 = w8a8.cutlass_w8a8_linear(x1.to(device), qw, sw, bias=None, workspace=ws, weight_t=qw.t(),
                                  weight_scale_t=sw.t())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits16(o1), _int8_reference(oracle, x1, w))
    o2 = w8a8.cutlass_w8a8_linear(x2.to(device), qw, sw, bias=None, workspace=ws, weight_t=None,
                                  weight_scale_t=None)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits16(o2), _int8_reference(oracle, x2, w))
    assert o1.data_ptr() == o2.data_ptr()
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        o3 = w8a8.cutlass_w8a8_linear(x2.to(device), qw, sw, bias=None, workspace=ws, weight_t=None,
                                      weight_scale_t=None)
    side.synchronize()
    assert o3.data_ptr() != o2.data_ptr()
    np.testing.assert_array_equal(bits16(o3), bits16(o2))


def test_model_level_int8_flow(oracle, device):
    """prepare slot -> stream load -> receipt -> workspace -> module forward,
    on a 7-block toy DiT (the policy keeps blocks 0, 1, 4, 5, 6 in bf16)."""
    w8a8 = _mod("inference.w8a8")
    model = _Transformer(device=device)
    names = w8a8.resolve_h3_cutlass_w8a8_policy(
        [n for n, _ in model.named_modules() if n.startswith("blocks.")], policy="interior_fc1_qkv_v1")
    assert names["quantized_linear_names"] == ["blocks.2.attn.qkv_proj", "blocks.2.mlp.fc1",
                                               "blocks.3.attn.qkv_proj", "blocks.3.mlp.fc1"]
    sources = {}
    for name in names["quantized_linear_names"]:
        module = model.get_submodule(name)
        sources[name] = module.weight.detach().cpu().clone()
        w8a8.prepare_cutlass_w8a8_stream_load_slot_(module, name=name)
        w8a8.load_cutlass_w8a8_stream_weight_(module, sources[name], name=name)
    receipt = w8a8.quantize_h3_interior_qkv_fc1_(model, policy="interior_fc1_qkv_v1")
    assert receipt["linear_count"] == 4 and receipt["post_load_conversion_linear_count"] == 0
    assert receipt["quantized_weight_bytes"] * 2 == receipt["source_weight_bytes"]
    assert w8a8.enable_h3_cutlass_w8a8_workspace_(model)["linear_count"] == 4
    assert all(ops_mod.is_tiled(model.get_submodule(n).weight) for n in names["quantized_linear_names"])
    for tokens in (2 * 96, 2 * 40, 7):   # large GEMM, then the weight-streaming GEMM (tiled activations)
        x = activations(tokens, 256, seed=12 + tokens, outlier_channels=2)
        for name in ("blocks.2.attn.qkv_proj", "blocks.3.mlp.fc1"):
            out = model.get_submodule(name)(x.reshape(1, tokens, 256).to(device))
            torch.cuda.synchronize()
            np.testing.assert_array_equal(bits16(out).reshape(tokens, -1),
                                          _int8_reference(oracle, x, sources[name]))


@pytest.mark.parametrize("fused", [False, True])
def test_fp8_tensor_quantizers(oracle, device, monkeypatch, fused):
    """Per-tensor quantizers in both reference modes: eager on the GPU (the
    divisor is the scale rounded to bf16) and with the fused Triton kernels
    enabled (fp32 divisor)."""
    fk = _mod("inference.fused_kernels")
    monkeypatch.setattr(fk, "_ENABLED", fused)
    x = activations(333, 1040, seed=4, outlier_channels=5)
    q, s = fk.quantize_fp8_e4m3_dynamic(x.to(device))
    rq, rs = oracle.quant_tensor_e4m3(bits16(x), bf16_divisor=not fused)
    np.testing.assert_array_equal(bits8(q), rq)
    assert s.dim() == 0 and np.float32(s.item()) == rs
    q2 = fk.quantize_fp8_e4m3(x.to(device), torch.tensor(0.0123, device=device))
    np.testing.assert_array_equal(bits8(q2), oracle.quant_tensor_e4m3(bits16(x), np.float32(0.0123),
                                                                      bf16_divisor=not fused)[0])
    # the eager expression evaluated by torch on the GPU is the unfused mode
    ref = torch.clamp(x.to(device) / s, -448.0, 448.0).to(torch.float8_e4m3fn)
    if not fused:
        np.testing.assert_array_equal(bits8(ref), bits8(q))
    q3, s3 = fk.quantize_fp8_e4m3_rowwise(x.reshape(9, 37, 1040).to(device))
    rq3, rs3 = oracle.quant_rows(bits16(x), "e4m3")
    assert tuple(s3.shape) == (9, 37, 1)
    np.testing.assert_array_equal(bits8(q3).reshape(333, 1040), rq3)
    np.testing.assert_array_equal(s3.cpu().numpy().ravel(), rs3)
    # fp32 input is quantized in its own dtype (fp32 quotient eager; bf16-rounded fused)
    q4, s4 = fk.quantize_fp8_e4m3_dynamic(x.float().to(device))
    rq4, rs4 = oracle.quant_tensor_e4m3_typed(x.float().numpy(), "f32", not fused)
    np.testing.assert_array_equal(bits8(q4), rq4)
    assert np.float32(s4.item()) == rs4
    with pytest.raises(TypeError):
        fk.quantize_fp8_e4m3_dynamic(x.to(torch.float64).to(device))


def test_fp8_w8a8_module_dispatch(oracle, device):
    """quantize_h3_block_linears_fp8_w8a8_ + the module forward vs the exact oracle."""
    fp8 = _mod("inference.fp8")
    model = _Transformer(device=device)
    originals = {n: m.weight.detach().cpu().clone() for n, m in model.named_modules()
                 if n.endswith(("qkv_proj", "out_proj", "fc1", "fc2"))}
    receipt = fp8.quantize_h3_block_linears_fp8_w8a8_(torch, model, policy="quality_first_residual_v1")
    assert receipt["linear_count"] == 2 * 2  # blocks 2..3 of 7: qkv and fc1 each
    assert model.get_submodule("blocks.3.attn.qkv_proj").weight.dtype == torch.float8_e4m3fn
    # fc2 of block 2 stays bf16 and runs F.linear
    fc2 = model.get_submodule("blocks.2.mlp.fc2")
    assert fc2.weight.dtype == torch.bfloat16
    fc1 = model.get_submodule("blocks.2.mlp.fc1")
    assert ops_mod.is_tiled(fc1.weight)
    rqw, rsw = oracle.quant_rows(bits16(originals["blocks.2.mlp.fc1"]), "e4m3")
    np.testing.assert_array_equal(bits8(fc1.weight), to_tiled(rqw))
    for tokens in (150, 48):   # large GEMM, then the weight-streaming GEMM
        xs = activations(tokens, 256, seed=7 + tokens, outlier_channels=3)
        out = fc1(xs.reshape(1, tokens, 256).to(device))
        torch.cuda.synchronize()
        assert tuple(out.shape) == (1, tokens, 512)
        rqa, rsa = oracle.quant_rows(bits16(xs), "e4m3")
        _assert_fp8_close(oracle, bits16(out).reshape(tokens, 512), rqa, rsa, rqw, rsw, None)


def test_fp8_per_tensor_module_dispatch(oracle, device):
    """Dynamic per-tensor FP8 block linear with bias (FL/distributed/linear.py:80-101)."""
    fp8 = _mod("inference.fp8")
    lin = _mod("distributed.linear")
    model = _Transformer(device=device)
    fc2 = model.get_submodule("blocks.3.mlp.fc2")
    bias = fc2.bias.detach().clone()
    weight = fc2.weight.detach().cpu().clone()
    receipt = fp8.quantize_h3_block_linears_dynamic_fp8_(torch, model)
    assert receipt["linear_count"] == 28 and receipt["weight_scale"] == "static_per_tensor"
    assert receipt["projection_set"] == "attention_and_mlp" and receipt["policy_rules"] is None
    assert receipt["activation_calibration_scope"] is None and receipt["base_model_bypass_forwards"] is None
    assert receipt["excluded_components"] == ["lora_adapter_tensors", "patch_projections", "timestep_projections",
                                              "final_output_projections", "token_refiner", "condition_and_adaln"]
    x = activations(130, 512, seed=9, outlier_channels=3)
    # eager mode (the fused kernels not enabled): bf16 divisors on the GPU
    rqa, rsa = oracle.quant_tensor_e4m3(bits16(x), bf16_divisor=True)
    rqw, rsw = oracle.quant_tensor_e4m3(bits16(weight), bf16_divisor=True)
    np.testing.assert_array_equal(bits8(fc2.weight), rqw)
    # row-parallel: partial output without bias, bias added after the reduction
    local = fc2.forward_local(x.to(device))
    torch.cuda.synchronize()
    _assert_fp8_close(oracle, bits16(local), rqa, np.array([rsa]), rqw, np.array([rsw]), None)
    # FL's functional form: the bias is fused into the scaled GEMM
    fused = lin._linear(x.to(device), fc2.weight, bias, fc2._fp8_weight_scale)
    torch.cuda.synchronize()
    _assert_fp8_close(oracle, bits16(fused), rqa, np.array([rsa]), rqw, np.array([rsw]), bits16(bias))


def test_fp8_calibrated_scale_then_static(oracle, device):
    """Calibration records the running max of amax/448; afterwards the frozen
    scale x margin is the static activation scale (FL/distributed/linear.py:104-128)."""
    fp8 = _mod("inference.fp8")
    model = _Transformer(blocks=5, device=device)
    receipt = fp8.quantize_h3_block_linears_calibrated_fp8_(torch, model, calibration_forwards=2, scale_margin=1.25)
    assert receipt["activation_calibration_scope"] == "student_av_forwards_only"
    assert receipt["base_model_bypass_forwards"] == "per_forward_scale_without_consuming_calibration"
    assert receipt["activation_scale"] == "calibrated_static_per_tensor"
    fc1 = model.get_submodule("blocks.1.mlp.fc1")
    xa = activations(64, 256, seed=1)
    xb = (activations(64, 256, seed=2).float() * 3).to(torch.bfloat16)
    fc1(xa.to(device))
    fc1(xb.to(device))
    torch.cuda.synchronize()
    amax = max(float(xa.float().abs().max()), float(xb.float().abs().max()))
    # torch evaluates tensor / 448.0 on the device as a multiply by RN(1/448)
    assert np.float32(fc1._fp8_activation_scale.item()) == np.float32(amax) * (np.float32(1.0) / np.float32(448.0))
    assert fc1._fp8_activation_calibration_remaining == 0
    xc = activations(64, 256, seed=3)
    static = np.float32(fc1._fp8_activation_scale.item() * np.float32(1.25))
    out = fc1(xc.to(device))
    torch.cuda.synchronize()
    rqa, _ = oracle.quant_tensor_e4m3(bits16(xc), static, bf16_divisor=True)
    rqw = bits8(fc1.weight)
    rsw = np.float32(fc1._fp8_weight_scale.item())
    _assert_fp8_close(oracle, bits16(out), rqa, np.array([static]), rqw, np.array([rsw]), None)


@pytest.mark.parametrize("fmt", ["int8", "fp8"])
def test_fused_lora_wrapper(oracle, device, fmt):
    """H3InferenceParallelLinearLoRA on a W8A8 base takes the fused path; the
    result is within a few bf16 ulps of the reference's three-rounding formula."""
    lora = _mod("inference.lora")
    w8a8 = _mod("inference.w8a8")
    from _toy_layers import ToyColumnLinear

    k, n, m, rank = 512, 384, 200, 64
    base = ToyColumnLinear(k, n, bias=False, dtype=torch.bfloat16, device=device)
    w = weights(n, k, seed=31)
    if fmt == "int8":
        qw, sw = w8a8._quantize_weight(w.to(device))
        base.weight = torch.nn.Parameter(qw, requires_grad=False)
        base.register_buffer("_cutlass_w8a8_weight_scale", sw, persistent=False)
    else:
        fp8 = _mod("inference.fp8")
        qw, sw = fp8.quantize_weight_fp8_rows(w.to(device))
        base.weight = torch.nn.Parameter(qw, requires_grad=False)
        base.register_buffer("_fp8_w8a8_weight_scale", sw, persistent=False)
    gen = torch.Generator().manual_seed(5)
    la = (torch.randn(rank, k, generator=gen) * 0.02).to(torch.bfloat16)
    lb = (torch.randn(n, rank, generator=gen) * 0.02).to(torch.bfloat16)
    wrapped = lora.H3InferenceParallelLinearLoRA(base, kind="column", a=la.to(device), b=lb.to(device), scale=0.75)
    x = activations(m, k, seed=32, outlier_channels=2)
    out = wrapped(x.to(device))
    base_out = base(x.to(device))
    torch.cuda.synchronize()
    ref = oracle.bf16_to_f32(oracle.lora_reference(bits16(x), bits16(la), bits16(lb), 0.75,
                                                   bits16(base_out))).astype(np.float64)
    got = oracle.bf16_to_f32(bits16(out)).astype(np.float64)
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 2.0 ** -7
    from _util import bf16_ulp

    assert np.max(np.abs(got - ref)) <= 4 * np.max(bf16_ulp(ref))


def test_fresh_transposed_view_of_a_tiled_weight(oracle, device):
    """A caller-made ``weight.t()`` of a tiled W8 parameter (allowed by
    H3/inference/w8a8.py:190-220) reaches the GEMM with the tiled layout:
    the layout is recorded against the storage, so every view carries it.
    A row-major call on that storage raises instead of reading tiled bytes."""
    w8a8 = _mod("inference.w8a8")
    k, n = 1024, 512
    m = torch.nn.Module()
    m.weight = torch.nn.Parameter(torch.empty(n, k, dtype=torch.bfloat16, device=device))
    m.bias = None
    w8a8.prepare_cutlass_w8a8_stream_load_slot_(m, name="blocks.2.mlp.fc1")
    w = weights(n, k, seed=41)
    w8a8.load_cutlass_w8a8_stream_weight_(m, w, name="blocks.2.mlp.fc1")
    assert ops_mod.is_tiled(m.weight) and ops_mod.is_tiled(m.weight.t()) and ops_mod.is_tiled(m.weight.data)
    x = activations(300, k, seed=42, outlier_channels=3)
    ref = _int8_reference(oracle, x, w)
    ws = w8a8.CutlassW8A8Workspace()
    for weight_t in (m.weight.t(), m.weight.detach().t(), None):
        out = w8a8.cutlass_w8a8_linear(x.to(device), m.weight, m._cutlass_w8a8_weight_scale, bias=None,
                                       workspace=ws, weight_t=weight_t, weight_scale_t=None)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bits16(out), ref)
    qa, sa = ops_mod.quant_rows(x.to(device), ops_mod.FMT_INT8, ops_mod.ROUND_RCP_MUL)
    with pytest.raises(ValueError, match="tiled codes"):
        ops_mod.scaled_mm(qa, m.weight.detach(), sa.reshape(-1), m._cutlass_w8a8_weight_scale.reshape(-1))
    # a copy is a new storage of row-major meaning: no tiled mark travels with it
    assert not ops_mod.is_tiled(m.weight.detach().clone())


def test_fl_w8a8_torch_first_api(oracle, device):
    """FL's twin (FL/inference/w8a8.py): post-load BF16 -> W8 conversion of the
    selected interior projections (validated before any change), the torch-first
    linear and workspace, and the streamed slot for a preallocated int8 weight."""
    fl = _mod("inference.fl_w8a8")
    assert fl.H3_CUTLASS_W8A8_POLICIES == ("interior_fc1_qkv_v1",)
    model = _Transformer(device=device)
    sources = {n: model.get_submodule(n).weight.detach().cpu().clone()
               for n in ("blocks.2.attn.qkv_proj", "blocks.3.mlp.fc1")}
    receipt = fl.quantize_h3_interior_qkv_fc1_linears_cutlass_w8a8_(torch, model, policy="interior_fc1_qkv_v1")
    assert receipt["linear_count"] == 4 and receipt["stream_load_linear_count"] == 0
    assert receipt["eligible_linear_count"] == 21 and receipt["bf16_boundary_block_indices"] == [0, 1, 4, 5, 6]
    assert receipt["quantized_linear_names"] == ["blocks.2.attn.qkv_proj", "blocks.2.mlp.fc1",
                                                 "blocks.3.attn.qkv_proj", "blocks.3.mlp.fc1"]
    assert 0.0 < receipt["eligible_weight_fraction"] < 1.0
    for name, w in sources.items():
        module = model.get_submodule(name)
        rq, rs = oracle.quant_rows(bits16(w), "int8", "div")
        assert ops_mod.is_tiled(module.weight)
        np.testing.assert_array_equal(bits8(module.weight), to_tiled(rq.view(np.uint8)))
        np.testing.assert_array_equal(module._cutlass_w8a8_weight_scale.cpu().numpy().ravel(), rs)
    # a repeated conversion finds complete storage... of the wrong kind: nothing changes
    with pytest.raises(RuntimeError, match="incomplete CUTLASS W8A8 storage"):
        fl.quantize_h3_interior_qkv_fc1_linears_cutlass_w8a8_(torch, model, policy="interior_fc1_qkv_v1")
    fc1 = model.get_submodule("blocks.3.mlp.fc1")
    x = activations(2 * 70, 256, seed=43, outlier_channels=2).reshape(2, 70, 256)
    out = fl.cutlass_w8a8_linear(torch, x.to(device), fc1.weight, fc1._cutlass_w8a8_weight_scale, bias=None)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits16(out).reshape(-1, 512),
                                  _int8_reference(oracle, x.reshape(-1, 256), sources["blocks.3.mlp.fc1"]))
    ws_receipt = fl.enable_h3_cutlass_w8a8_workspace_(torch, model)
    assert ws_receipt["linear_count"] == 4 and ws_receipt["arithmetic_order_changed"] is False
    out_ws = model.get_submodule("blocks.3.mlp.fc1")(x.to(device))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits16(out_ws), bits16(out))
    # streamed slot on a preallocated, frozen int8 weight (FL layers allocate it at construction)
    slot = torch.nn.Module()
    slot.weight = torch.nn.Parameter(torch.empty(64, 256, dtype=torch.int8, device=device), requires_grad=False)
    slot.bias = None
    fl.prepare_cutlass_w8a8_stream_load_slot_(torch, slot, name="blocks.2.mlp.fc1")
    src = weights(64, 256, seed=44)
    fl.load_cutlass_w8a8_stream_weight_(torch, slot, src, name="blocks.2.mlp.fc1", maximum_temporary_bytes=4096)
    torch.cuda.synchronize()
    rq, rs = oracle.quant_rows(bits16(src), "int8", "div")
    np.testing.assert_array_equal(bits8(slot.weight), to_tiled(rq.view(np.uint8)))
    np.testing.assert_array_equal(slot._cutlass_w8a8_weight_scale.cpu().numpy().ravel(), rs)
    with pytest.raises(RuntimeError, match="already owns CUTLASS W8A8 storage"):
        fl.prepare_cutlass_w8a8_stream_load_slot_(torch, slot, name="blocks.2.mlp.fc1")


def test_lora_adapter_switch_on_a_quantized_base(device):
    """With the adapter switched off the wrapper returns exactly the W8A8 base output."""
    lora = _mod("inference.lora")
    w8a8 = _mod("inference.w8a8")
    from _toy_layers import ToyColumnLinear

    k, n, rank = 512, 256, 32
    base = ToyColumnLinear(k, n, bias=False, dtype=torch.bfloat16, device=device)
    qw, sw = w8a8._quantize_weight(weights(n, k, seed=45).to(device))
    base.weight = torch.nn.Parameter(qw, requires_grad=False)
    base.register_buffer("_cutlass_w8a8_weight_scale", sw, persistent=False)
    gen = torch.Generator().manual_seed(46)
    la = (torch.randn(rank, k, generator=gen) * 0.02).to(torch.bfloat16).to(device)
    lb = (torch.randn(n, rank, generator=gen) * 0.02).to(torch.bfloat16).to(device)
    wrapped = lora.H3InferenceParallelLinearLoRA(base, kind="column", a=la, b=lb, scale=1.0)
    x = activations(96, k, seed=47, outlier_channels=2).to(device)
    with_adapter = wrapped(x)
    wrapped.adapter_enabled = False
    without = wrapped(x)
    torch.cuda.synchronize()
    assert torch.equal(without, base(x))
    assert not torch.equal(with_adapter, without)


@pytest.mark.parametrize("scale", [1.0, 0.75])
@pytest.mark.parametrize("tokens", [(2, 150), (1, 96)])
def test_reference_lora_wrappers_swapped_to_fused_epilogue(oracle, device, monkeypatch, scale, tokens):
    """The drop-in path of the LoRA epilogue: wrappers shaped like the ones the
    reference's apply_h3_lora_checkpoint installs (H3/inference/lora_checkpoint.py:
    172-246; fp32 buffers) on int8 W8A8 bases (FL/inference/w8a8.py:340-466
    post-load conversion through ``getattr(module, "base", module)``), bf16
    buffers materialised (:261-284), then fuse_h3_lora_wrappers_.  The swapped
    wrappers on W8A8 bases take the fused GEMM epilogue and agree with the
    reference's three rounding points (:196-205) to 4 bf16 ulps; the one on a
    bf16 base keeps the reference's formula bit for bit."""
    from _toy_layers import install_reference_lora

    fl = _mod("inference.fl_w8a8")
    lora = _mod("inference.lora")
    model = _Transformer(device=device)
    targets = ["blocks.2.attn.qkv_proj", "blocks.3.mlp.fc1", "blocks.0.attn.qkv_proj"]
    installed = install_reference_lora(model, targets, rank=128, scale=scale, seed=61)
    fl.quantize_h3_interior_qkv_fc1_linears_cutlass_w8a8_(torch, model, policy="interior_fc1_qkv_v1")
    lora.materialize_h3_lora_bf16_buffers_(model)
    x = activations(tokens[0] * tokens[1], 256, seed=62, outlier_channels=2).reshape(*tokens, 256).to(device)
    before = {name: installed[name](x) for name in targets}
    receipt = lora.fuse_h3_lora_wrappers_(model)
    assert receipt["replaced_count"] == 3 and receipt["fused_epilogue_ready_count"] == 2
    calls = []
    fused = lora.fused_quantized_lora_linear
    monkeypatch.setattr(lora, "fused_quantized_lora_linear", lambda *a: calls.append(1) or fused(*a))
    after = {name: model.get_submodule(name)(x) for name in targets}
    torch.cuda.synchronize()
    assert len(calls) == 2
    from _util import bf16_ulp

    flat = bits16(x.reshape(-1, 256))
    for name in targets[:2]:
        wrapper = model.get_submodule(name)
        assert isinstance(wrapper, lora.H3InferenceParallelLinearLoRA)
        assert wrapper.lora_a is installed[name].lora_a and wrapper.lora_a.dtype == torch.bfloat16
        n = int(wrapper.base.weight.shape[0])
        base_out = bits16(wrapper.base(x).reshape(-1, n))
        ref = oracle.bf16_to_f32(oracle.lora_reference(flat, bits16(wrapper.lora_a), bits16(wrapper.lora_b), scale,
                                                       base_out)).astype(np.float64)
        base_f = oracle.bf16_to_f32(base_out).astype(np.float64)
        # one rounding against three: 4 ulps of the largest of output, base and update
        bound = 4 * bf16_ulp(np.maximum(np.maximum(np.abs(ref), np.abs(base_f)), np.abs(ref - base_f)))
        for got_t in (after[name], before[name]):
            got = oracle.bf16_to_f32(bits16(got_t.reshape(-1, n))).astype(np.float64)
            assert np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 2.0 ** -7
            assert np.all(np.abs(got - ref) <= bound)
    assert torch.equal(after[targets[2]], before[targets[2]])


def test_deepcopy_of_a_tiled_w8a8_model(device):
    """copy.deepcopy of a model whose W8 weights are stored tiled (FL's
    post-load conversion, then the workspace with its precomputed weight_t
    views): the copy's projections return the original's bits."""
    import copy

    fl = _mod("inference.fl_w8a8")
    model = _Transformer(device=device)
    fl.quantize_h3_interior_qkv_fc1_linears_cutlass_w8a8_(torch, model, policy="interior_fc1_qkv_v1")
    fl.enable_h3_cutlass_w8a8_workspace_(torch, model)
    twin = copy.deepcopy(model)
    for rows in (300, 64):
        x = activations(rows, 256, seed=63 + rows, outlier_channels=2).to(device)
        for name in ("blocks.2.attn.qkv_proj", "blocks.3.mlp.fc1"):
            ref = model.get_submodule(name)(x).clone()
            got = twin.get_submodule(name)(x)
            torch.cuda.synchronize()
            assert torch.equal(got, ref), name
    assert ops_mod.is_tiled(twin.get_submodule("blocks.3.mlp.fc1").weight)
