"""GPU parity of the scaled GEMMs against the CPU oracle.

* int8: int32 accumulators bit-exact; bf16 outputs bit-exact against the
  oracle epilogue s_a * (s_w * float(acc)) [fma with bias].
* e4m3: against the exact (binary64) dot products.  Bound per element:
      |got - ref| <= ulp_bf16(ref) + K * 2^-24 * s_a * s_w * sum_k |a_k b_k|
  (one bf16 rounding on each side plus the worst case of a binary32
  accumulation of K products), and relative Frobenius error <= 2^-8.
* LoRA epilogue and down-projection: against the reference rounding points
  (H3/inference/lora_checkpoint.py:196-205) with a bf16-level tolerance.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _util import activations, bf16_ulp, bits16, bits8, fp32_gemm_bound, weights

pytestmark = pytest.mark.gpu


def _rand_i8(shape, seed, extremes=False):
    gen = torch.Generator().manual_seed(seed)
    t = torch.randint(-127, 128, shape, generator=gen, dtype=torch.int32)
    if extremes:
        t[: shape[0] // 4] = 127
        t[shape[0] // 4: shape[0] // 2] = -128
    return t.to(torch.int8)


@pytest.mark.parametrize("m,n,k", [(256, 256, 128), (300, 200, 1040), (256, 1024, 1024), (33, 17, 16),
                                   (512, 768, 5120)])
def test_int8_accumulators_bit_exact(ops, oracle, device, m, n, k):
    print(f"i32 gemm {m}x{n}x{k}", flush=True)
    a = _rand_i8((m, k), 1)
    b = _rand_i8((n, k), 2)
    c = ops.gemm_i8_i32(a.to(device), b.to(device))
    torch.cuda.synchronize()
    ref = oracle.gemm_i8_i32_fast(a.numpy(), b.numpy())
    np.testing.assert_array_equal(c.cpu().numpy(), ref)


def test_int8_accumulator_extremes(ops, oracle, device):
    """Largest accumulators at K = 13824 (c3 down): rows of +127 / -128
    against rows of +127 / -128 reach 128^2 * K = 2.26e8 (< 2^31)."""
    k = 13824
    a = _rand_i8((64, k), 3, extremes=True)
    b = _rand_i8((64, k), 4, extremes=True)
    c = ops.gemm_i8_i32(a.to(device), b.to(device))
    torch.cuda.synchronize()
    ref = oracle.gemm_i8_i32_fast(a.numpy(), b.numpy())
    assert np.abs(ref).max() >= 127 * 128 * k
    np.testing.assert_array_equal(c.cpu().numpy(), ref)


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("m,n,k", [(256, 1024, 1024), (100, 300, 2048), (640, 512, 5120)])
def test_int8_scaled_bit_exact(ops, oracle, device, m, n, k, bias):
    x = activations(m, k, seed=m, outlier_channels=8)
    w = weights(n, k, seed=n)
    xg, wg = x.to(device), w.to(device)
    qw, sw = ops.quant_rows(wg, ops.FMT_INT8, ops.ROUND_DIV)
    qa, sa = ops.quant_rows(xg, ops.FMT_INT8, ops.ROUND_RCP_MUL)
    bvec = (torch.randn(n, generator=torch.Generator().manual_seed(9)) * 0.01).to(torch.bfloat16)
    out = ops.scaled_mm(qa, qw, sa, sw, bias=bvec.to(device) if bias else None)
    torch.cuda.synchronize()
    rqa, rsa = oracle.quant_rows(bits16(x), "int8", "rcp")
    rqw, rsw = oracle.quant_rows(bits16(w), "int8", "div")
    acc = oracle.gemm_i8_i32_fast(rqa, rqw)
    ref = oracle.epilogue(acc, rsa, rsw, bits16(bvec) if bias else None)
    np.testing.assert_array_equal(bits16(out), ref)


def _fp8_case(ops, oracle, device, m, n, k, seed, bias, per_tensor=False):
    x = activations(m, k, seed=seed, outlier_channels=max(1, k // 100), outlier_scale=15.0)
    w = weights(n, k, seed=seed + 1)
    xg, wg = x.to(device), w.to(device)
    if per_tensor:
        qa, sa = ops.quant_tensor_e4m3(xg)
        qw, sw = ops.quant_tensor_e4m3(wg)
        rqa, rsa = oracle.quant_tensor_e4m3(bits16(x))
        rqw, rsw = oracle.quant_tensor_e4m3(bits16(w))
        rsa, rsw = np.array([rsa]), np.array([rsw])
    else:
        qa, sa = ops.quant_rows(xg, ops.FMT_E4M3FN)
        qw, sw = ops.quant_rows(wg, ops.FMT_E4M3FN)
        rqa, rsa = oracle.quant_rows(bits16(x), "e4m3")
        rqw, rsw = oracle.quant_rows(bits16(w), "e4m3")
    bvec = (torch.randn(n, generator=torch.Generator().manual_seed(seed + 2)) * 0.01).to(torch.bfloat16)
    out = ops.scaled_mm(qa, qw, sa.reshape(-1), sw.reshape(-1), bias=bvec.to(device) if bias else None)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits8(qa), rqa)
    np.testing.assert_array_equal(bits8(qw), rqw)
    return out, rqa, rsa, rqw, rsw, (bits16(bvec) if bias else None)


def _assert_fp8_close(oracle, got_bits, rqa, rsa, rqw, rsw, bias_bits, rows=None):
    if rows is not None:
        rqa = rqa[rows]
        rsa = rsa[rows] if rsa.size > 1 else rsa
        got_bits = got_bits[rows]
    exact = oracle.gemm_e4m3_exact_fast(rqa, rqw)
    ref = oracle.bf16_to_f32(oracle.epilogue(exact, rsa, rsw, bias_bits)).astype(np.float64)
    got = oracle.bf16_to_f32(got_bits).astype(np.float64)
    lut = oracle.e4m3_lut().astype(np.float64)
    abs_sum = np.abs(lut[rqa]) @ np.abs(lut[rqw]).T
    scale = np.ravel(rsa).astype(np.float64)[:, None] * np.ravel(rsw).astype(np.float64)[None, :]
    k = rqa.shape[1]
    bound = bf16_ulp(ref) + fp32_gemm_bound(k, abs_sum * scale) + 1e-30
    err = np.abs(got - ref)
    worst = np.argmax(err / bound)
    assert np.all(err <= bound), f"max err/bound {(err / bound).max():.3f} at {np.unravel_index(worst, err.shape)}"
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert rel <= 2.0 ** -8, rel


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("m,n,k", [(256, 1024, 1024), (300, 200, 1040), (1, 256, 512), (640, 768, 5120),
                                   (257, 511, 13824)])
def test_fp8_scaled_matches_exact(ops, oracle, device, m, n, k, bias):
    print(f"fp8 gemm {m}x{n}x{k} bias={bias}", flush=True)
    out, rqa, rsa, rqw, rsw, bb = _fp8_case(ops, oracle, device, m, n, k, seed=m + n + k, bias=bias)
    _assert_fp8_close(oracle, bits16(out), rqa, rsa, rqw, rsw, bb)


def test_fp8_per_tensor_scales(ops, oracle, device):
    out, rqa, rsa, rqw, rsw, bb = _fp8_case(ops, oracle, device, 384, 640, 2048, seed=11, bias=True,
                                            per_tensor=True)
    _assert_fp8_close(oracle, bits16(out), rqa, rsa, rqw, rsw, bb)


def test_fp8_c2_shape_sampled_rows(ops, oracle, device):
    """BASELINE c2 (QKV 480p: M=8192, K=5120, N=15360): full GPU GEMM, 48
    seeded rows checked against the exact oracle across all N columns."""
    out, rqa, rsa, rqw, rsw, bb = _fp8_case(ops, oracle, device, 8192, 15360, 5120, seed=0, bias=True)
    rows = np.sort(np.random.default_rng(0).choice(8192, 48, replace=False))
    _assert_fp8_close(oracle, bits16(out), rqa, rsa, rqw, rsw, bb, rows=rows)


@pytest.mark.parametrize("m,n,k,rank", [(256, 512, 1024, 128), (300, 200, 1040, 128), (64, 256, 512, 64)])
def test_fp8_lora_epilogue(ops, oracle, device, m, n, k, rank):
    """Fused LoRA slab vs. the reference rounding points: the fused result
    rounds once, the reference rounds base, t@B^T and the sum separately,
    so they may differ by a few bf16 ulps of the output."""
    out0, rqa, rsa, rqw, rsw, bb = _fp8_case(ops, oracle, device, m, n, k, seed=21, bias=False)
    x = activations(m, k, seed=21, outlier_channels=max(1, k // 100), outlier_scale=15.0)
    gen = torch.Generator().manual_seed(5)
    la = (torch.randn(rank, k, generator=gen) * 0.01).to(torch.bfloat16)
    lb = (torch.randn(n, rank, generator=gen) * 0.01).to(torch.bfloat16)
    xg = x.to(device)
    qa, sa = ops.quant_rows(xg, ops.FMT_E4M3FN)
    qw, sw = ops.quant_rows(weights(n, k, seed=22).to(device), ops.FMT_E4M3FN)
    t = ops.lora_down(xg, la.to(device))
    out = ops.scaled_mm(qa, qw, sa, sw, lora_t=t, lora_b=lb.to(device), lora_scale=1.0)
    torch.cuda.synchronize()
    # t itself: bf16(x @ A^T) within one bf16 rounding of the binary32 sum
    t_ref = oracle.lora_down_reference(bits16(x), bits16(la))
    t_got = oracle.bf16_to_f32(bits16(t)).astype(np.float64)
    absx = np.abs(oracle.bf16_to_f32(bits16(x)).astype(np.float64))
    absa = np.abs(oracle.bf16_to_f32(bits16(la)).astype(np.float64))
    t_bound = bf16_ulp(t_ref) + fp32_gemm_bound(k, absx @ absa.T)
    assert np.all(np.abs(t_got - t_ref) <= t_bound)
    base = oracle.epilogue(oracle.gemm_e4m3_exact_fast(bits8(qa), bits8(qw)), sa.cpu().numpy(), sw.cpu().numpy())
    ref = oracle.bf16_to_f32(oracle.lora_reference(bits16(x), bits16(la), bits16(lb), 1.0, base)).astype(np.float64)
    got = oracle.bf16_to_f32(bits16(out)).astype(np.float64)
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert rel <= 2.0 ** -7, rel
    assert np.max(np.abs(got - ref)) <= 4 * np.max(bf16_ulp(ref)), np.max(np.abs(got - ref))


def test_int8_layout_identity(ops, device):
    """A = I (identity codes) picks out rows of B: checks the MFMA operand and
    accumulator lane layouts independently of any arithmetic tolerance."""
    k = 256
    a = torch.zeros(k, k, dtype=torch.int8)
    a[torch.arange(k), torch.arange(k)] = 1
    b = _rand_i8((320, k), 8)
    c = ops.gemm_i8_i32(a.to(device), b.to(device))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(c.cpu().numpy(), b.numpy().astype(np.int32).T)


def test_fp8_layout_identity(ops, device):
    k = 256
    one = 0x38  # e4m3fn 1.0
    a = torch.zeros(k, k, dtype=torch.uint8)
    a[torch.arange(k), torch.arange(k)] = one
    gen = torch.Generator().manual_seed(4)
    b = torch.randint(0, 0x7E, (288, k), generator=gen, dtype=torch.int32).to(torch.uint8)
    ones = torch.ones(k, dtype=torch.float32)
    out = ops.scaled_mm(a.view(torch.float8_e4m3fn).to(device), b.view(torch.float8_e4m3fn).to(device),
                        ones.to(device), torch.ones(288, device=device))
    torch.cuda.synchronize()
    expect = b.view(torch.float8_e4m3fn).float().t().to(torch.bfloat16)
    assert torch.equal(out.cpu(), expect)
