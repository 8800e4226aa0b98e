"""FP8DynamicLinear's path on the GPU: per-tensor quantization of fp16 and
fp32 tensors in their own dtype, and the scaled GEMM's binary16 epilogue.

References: FL/inference/fp8.py:96-146 (FP8DynamicLinear: weight quantized
in its dtype, fp16 bias, torch._scaled_mm(out_dtype=float16)),
FL/inference/fused_kernels.py:771-820 (eager and Triton quantizers).
"""

from __future__ import annotations

import importlib

import numpy as np
import pytest
import torch

from _util import activations, bits16, bits8, weights

pytestmark = pytest.mark.gpu

_DT = {"f16": torch.float16, "f32": torch.float32}


def _bits(x: torch.Tensor) -> np.ndarray:
    """Host bits of an fp16 tensor (uint16) or the fp32 values."""
    x = x.detach().cpu().contiguous()
    return x.view(torch.int16).numpy().view(np.uint16) if x.dtype == torch.float16 else x.numpy()


def _inputs(m: int, k: int, seed: int, dtype: str) -> torch.Tensor:
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=gen) * torch.exp2(torch.randint(-8, 4, (1, k), generator=gen).float())
    x[:, : max(1, k // 100)] *= 30.0
    return x.to(_DT[dtype])


@pytest.mark.parametrize("dtype", ["f16", "f32"])
@pytest.mark.parametrize("eager", [True, False])
@pytest.mark.parametrize("static", [False, True])
@pytest.mark.parametrize("m,k", [(40, 384), (3, 37), (2500, 256), (1030, 1001)])
def test_typed_tensor_quant_matches_oracle(ops, oracle, device, dtype, eager, static, m, k):
    print(f"typed per-tensor {dtype} eager={eager} static={static} {m}x{k}", flush=True)
    x = _inputs(m, k, m + k, dtype)
    st = 0.0371 if static else None
    sg = torch.tensor(st, dtype=torch.float32, device=device) if static else None
    q, s = ops.quant_tensor_e4m3(x.to(device), sg, eager=eager)
    torch.cuda.synchronize()
    rq, rs = oracle.quant_tensor_e4m3_typed(_bits(x), dtype, eager, st)
    assert np.float32(s.item()) == rs
    np.testing.assert_array_equal(bits8(q), rq)


@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_typed_tensor_quant_is_the_reference_expression_on_the_device(ops, device, dtype):
    """torch evaluates the reference's eager expression on this GPU
    (FL/inference/fused_kernels.py:791-796); the kernel gives its bits."""
    x = _inputs(300, 512, 7, dtype).to(device)
    scale = torch.clamp(x.detach().abs().amax().to(torch.float32) / 448.0, min=1.0e-12)
    ref = torch.clamp(x / scale, -448.0, 448.0).to(torch.float8_e4m3fn)
    q, s = ops.quant_tensor_e4m3(x, eager=True)
    torch.cuda.synchronize()
    assert s.item() == scale.item()
    np.testing.assert_array_equal(bits8(q), bits8(ref))


@pytest.mark.parametrize("dtype", ["f16", "f32"])
@pytest.mark.parametrize("static", [False, True])
def test_typed_tensor_quant_infinities_and_nans_on_the_device(ops, oracle, device, dtype, static):
    """With infinities and a NaN in the tensor: the reference's eager
    expression evaluated by torch on this GPU, the kernel and the oracle
    agree (a dynamic scale is NaN, every code NaN; under a static scale the
    infinities saturate to +-448 and the NaN stays NaN).  NaN codes are
    compared as NaN."""
    x = _inputs(300, 512, 9, dtype)
    x[7, 3] = float("inf")
    x[100, 500] = float("-inf")
    x[250, 0] = float("nan")
    xd = x.to(device)
    st = 0.0371 if static else None
    if static:
        scale = torch.tensor(st, dtype=torch.float32, device=device)
        q, s = ops.quant_tensor_e4m3(xd, scale, eager=True)
    else:
        scale = torch.clamp(xd.detach().abs().amax().to(torch.float32) / 448.0, min=1.0e-12)
        q, s = ops.quant_tensor_e4m3(xd, eager=True)
    ref = torch.clamp(xd / scale, -448.0, 448.0).to(torch.float8_e4m3fn)
    torch.cuda.synchronize()
    rq, rs = oracle.quant_tensor_e4m3_typed(_bits(x), dtype, True, st)
    for sv in (scale.item(), rs):
        assert (np.isnan(s.item()) and np.isnan(sv)) or s.item() == sv
    got = bits8(q)
    for want in (bits8(ref), rq):
        nan_q = (want & 0x7F) == 0x7F
        np.testing.assert_array_equal((got & 0x7F) == 0x7F, nan_q)
        np.testing.assert_array_equal(np.where(nan_q, 0, got), np.where(nan_q, 0, want))


def test_typed_tensor_quant_all_zero_fp16(ops, device):
    """fp16(1e-12) == 0: the eager quotient is 0 / 0 and every code is NaN,
    as in the reference.  The NaN's sign is the device's: the reference's
    CUDA device produces the positive canonical NaN (code 0x7F), which the
    kernel and the oracle write; torch on MI355X divides to a negative NaN
    (0xFF).  fp32 zeros give zero codes."""
    z = torch.zeros(5, 64, dtype=torch.float16, device=device)
    ref = torch.clamp(z / torch.clamp(z.abs().amax().float() / 448.0, min=1e-12), -448.0, 448.0)
    ref = ref.to(torch.float8_e4m3fn)
    q, _ = ops.quant_tensor_e4m3(z, eager=True)
    torch.cuda.synchronize()
    assert np.all(bits8(ref) & 0x7F == 0x7F)
    assert np.all(bits8(q) == 0x7F)
    q32, _ = ops.quant_tensor_e4m3(z.float(), eager=True)
    torch.cuda.synchronize()
    assert np.all(bits8(q32) == 0)


def test_typed_bf16_takes_the_bf16_quantizer(ops, device):
    x = activations(777, 1024, seed=4, outlier_channels=9).to(device)
    for eager in (False, True):
        q, s = ops.quant_tensor_e4m3(x, eager=eager)
        q0, s0 = ops.quant_tensor_e4m3(x, bf16_divisor=eager)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bits8(q), bits8(q0))
        assert s.item() == s0.item()


def f16_ulp(v: np.ndarray) -> np.ndarray:
    """Spacing of binary16 values at |v| (11 significant bits, subnormal below 2^-14)."""
    a = np.abs(v.astype(np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -14)))
    return 2.0 ** (e - 10)


def _assert_fp8_f16_close(oracle, got_bits, rqa, rsa, rqw, rsw, bias_bits):
    """The binary16 twin of the bf16 check: the oracle's model of the FP8
    instruction through the fp16 epilogue; per element within one fp16 ulp
    plus the model's combination bound times the scales plus 2^-22 relative;
    99% bit-identical."""
    model, rbound = oracle.gemm_e4m3_mfma(rqa, rqw)
    ref_bits = oracle.epilogue(model, rsa, rsw, bias_bits, out_f16=True)
    ref = oracle.f16_to_f32(ref_bits).astype(np.float64)
    got = oracle.f16_to_f32(got_bits).astype(np.float64)
    scale = np.abs(np.ravel(rsa).astype(np.float64))[:, None] * np.abs(np.ravel(rsw).astype(np.float64))[None, :]
    bound = f16_ulp(np.maximum(np.abs(ref), np.abs(got))) + rbound * scale + 2.0 ** -22 * np.abs(ref) + 1e-30
    err = np.abs(got - ref)
    assert np.all(err <= bound), f"max err/bound {(err / bound).max():.3f}"
    same = float(np.mean(got_bits == ref_bits))
    print(f"bit-identical to the model: {same:.5f}", flush=True)
    if got.size >= 1000:
        assert same >= 0.99, same


# Shapes by kernel: four-wave (512 x 1024 x 1024), persistent (n % 8 != 0),
# tile (k % 128 != 0), weight-streaming (m <= 128).
_F16_SHAPES = [(512, 1024, 1024), (300, 1004, 1024), (300, 200, 1040), (16, 512, 1024), (100, 96, 256)]


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("m,n,k", _F16_SHAPES)
def test_e4m3_f16_output(ops, oracle, device, m, n, k, bias):
    """Per-tensor e4m3 codes (the FP8DynamicLinear form) with an fp16 bias,
    rounded once to fp16."""
    print(f"e4m3 -> f16 {m}x{n}x{k} bias={bias}", flush=True)
    x = _inputs(m, k, m, "f16")
    w = _inputs(n, k, n + 1, "f32") * 0.02
    qa, sa = ops.quant_tensor_e4m3(x.to(device), eager=True)
    qw, sw = ops.quant_tensor_e4m3(w.to(device), eager=True)
    bvec = (torch.randn(n, generator=torch.Generator().manual_seed(3)) * 0.5).to(torch.float16)
    out = ops.scaled_mm(qa, qw, sa.reshape(1), sw.reshape(1), bias=bvec.to(device) if bias else None,
                        out_dtype=torch.float16)
    torch.cuda.synchronize()
    assert out.dtype == torch.float16
    rqa, rsa = oracle.quant_tensor_e4m3_typed(_bits(x), "f16", True)
    rqw, rsw = oracle.quant_tensor_e4m3_typed(_bits(w), "f32", True)
    np.testing.assert_array_equal(bits8(qa), rqa)
    np.testing.assert_array_equal(bits8(qw), rqw)
    _assert_fp8_f16_close(oracle, bits16(out), rqa, np.array([rsa]), rqw, np.array([rsw]),
                          _bits(bvec) if bias else None)


@pytest.mark.parametrize("m,n,k", [(256, 1024, 1024), (100, 300, 2048), (16, 512, 1040)])
def test_int8_f16_output_bit_exact(ops, oracle, device, m, n, k):
    x = activations(m, k, seed=m, outlier_channels=8)
    w = weights(n, k, seed=n)
    qa, sa = ops.quant_rows(x.to(device), ops.FMT_INT8, ops.ROUND_RCP_MUL)
    qw, sw = ops.quant_rows(w.to(device), ops.FMT_INT8, ops.ROUND_DIV)
    bvec = (torch.randn(n, generator=torch.Generator().manual_seed(9)) * 0.01).to(torch.float16)
    out = ops.scaled_mm(qa, qw, sa, sw, bias=bvec.to(device), out_dtype=torch.float16)
    torch.cuda.synchronize()
    rqa, rsa = oracle.quant_rows(bits16(x), "int8", "rcp")
    rqw, rsw = oracle.quant_rows(bits16(w), "int8", "div")
    ref = oracle.epilogue(oracle.gemm_i8_i32_fast(rqa, rqw), rsa, rsw, _bits(bvec), out_f16=True)
    np.testing.assert_array_equal(bits16(out), ref)


def test_scaled_mm_f16_checks(ops, device):
    qa = torch.zeros(4, 64, dtype=torch.float8_e4m3fn, device=device)
    one = torch.ones(1, device=device)
    with pytest.raises(ValueError, match="float16 vector"):
        ops.scaled_mm(qa, qa, one, one, bias=torch.zeros(4, dtype=torch.bfloat16, device=device),
                      out_dtype=torch.float16)
    with pytest.raises(TypeError, match="out_dtype"):
        ops.scaled_mm(qa, qa, one, one, out_dtype=torch.float32)


@pytest.mark.parametrize("fused", [False, True])
def test_fp8_dynamic_linear_module(oracle, device, monkeypatch, fused):
    """quantize_aligned_linears_dynamic_fp8_ on fp32 Linears (the VAE's
    dtype) fed fp16 activations: weight codes in fp32 (eager), activation
    codes in fp16 (eager) or bf16-rounded (fused kernels on), fp16 bias and
    output (FL/inference/fp8.py:96-183)."""
    fp8 = importlib.import_module("taomate_h3_amd.inference.fp8")
    fk = importlib.import_module("taomate_h3_amd.inference.fused_kernels")
    monkeypatch.setattr(fk, "_ENABLED", fused)
    torch.manual_seed(0)
    model = torch.nn.Sequential(torch.nn.Linear(256, 512), torch.nn.SiLU(), torch.nn.Linear(512, 96, bias=False),
                                torch.nn.Linear(96, 50)).to(device)
    w0 = model[0].weight.detach().cpu().clone()
    b0 = model[0].bias.detach().cpu().clone()
    receipt = fp8.quantize_aligned_linears_dynamic_fp8_(torch, model)
    assert receipt["linear_count"] == 2  # 96 -> 50 is not 16-aligned
    assert isinstance(model[3], torch.nn.Linear)
    lin = model[0]
    rqw, rsw = oracle.quant_tensor_e4m3_typed(w0.numpy(), "f32", True)
    np.testing.assert_array_equal(bits8(lin.weight), rqw)
    assert lin.weight_scale.item() == rsw and lin.bias.dtype == torch.float16
    x = _inputs(2 * 40, 256, 11, "f16").reshape(2, 40, 256)
    out = lin(x.to(device))
    torch.cuda.synchronize()
    assert out.shape == (2, 40, 512) and out.dtype == torch.float16
    rqa, rsa = oracle.quant_tensor_e4m3_typed(_bits(x.reshape(80, 256)), "f16", not fused)
    _assert_fp8_f16_close(oracle, bits16(out.reshape(80, 512)), rqa, np.array([rsa]), rqw, np.array([rsw]),
                          _bits(b0.to(torch.float16)))
