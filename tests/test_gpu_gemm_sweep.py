"""Seeded sweep of the scaled int8 GEMM over ragged shapes, layouts and
output strides: every output bit-exact against the oracle epilogue of the
exact int32 accumulators (the int8 W8A8 linear, H3/inference/w8a8.py:179-186).

The shapes cover the weight-streaming kernel (m <= 128), the four-wave kernel
with whole and half tiles, and the row-major fallbacks (k not a multiple of
128); n and m are ragged against every tile size, and some outputs are
strided views whose rows do not allow vector stores."""

from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from _util import activations, bits8, bits16, weights

pytestmark = pytest.mark.gpu


def _cases(count: int = 32, seed: int = 20261202):
    rng = random.Random(seed)
    out = []
    while len(out) < count:
        m = rng.choice([rng.randint(1, 128), rng.randint(129, 600)])
        n = rng.randint(1, 700)
        b_tiled = rng.random() < 0.6
        a_tiled = b_tiled and rng.random() < 0.5
        k = 128 * rng.randint(1, 16) if b_tiled or rng.random() < 0.5 else 16 * rng.randint(1, 128)
        if m * n * k > 3e8:
            continue
        pad = rng.choice([0, 0, 3, 8])
        if a_tiled and m > 128:  # tiled activations past the skinny rows: the four-wave kernel's shapes only
            n, k, pad = (n + 7) // 8 * 8, max(k, 256), pad // 8 * 8
        out.append((m, n, k, a_tiled, b_tiled, rng.random() < 0.5, pad))
    return out


@pytest.mark.parametrize("m,n,k,a_tiled,b_tiled,bias,pad", _cases())
def test_int8_sweep_bit_exact(ops, oracle, device, m, n, k, a_tiled, b_tiled, bias, pad):
    print(f"int8 sweep {m}x{n}x{k} a_tiled={a_tiled} b_tiled={b_tiled} bias={bias} ldo=n+{pad}", flush=True)
    x = activations(m, k, seed=m + k, outlier_channels=max(1, k // 100), outlier_scale=15.0)
    w = weights(n, k, seed=n + k)
    xg, wg = x.to(device), w.to(device)
    qw, sw = (ops.quant_rows_tiled if b_tiled else ops.quant_rows)(wg, ops.FMT_INT8, ops.ROUND_DIV)
    qa, sa = (ops.quant_rows_tiled if a_tiled else ops.quant_rows)(xg, ops.FMT_INT8, ops.ROUND_RCP_MUL)
    bvec = (torch.randn(n, generator=torch.Generator().manual_seed(n)) * 0.01).to(torch.bfloat16)
    big = torch.full((m, n + pad), float("nan"), device=device, dtype=torch.bfloat16)
    out = big[:, :n]
    ops.scaled_mm(qa, qw, sa.reshape(-1), sw.reshape(-1), bias=bvec.to(device) if bias else None, out=out,
                  a_tiled=a_tiled, b_tiled=b_tiled, m=m, n=n)
    torch.cuda.synchronize()
    rqa, rsa = oracle.quant_rows(bits16(x), "int8", "rcp")
    rqw, rsw = oracle.quant_rows(bits16(w), "int8", "div")
    ref = oracle.epilogue(oracle.gemm_i8_i32_fast(rqa, rqw), rsa, rsw, bits16(bvec) if bias else None)
    np.testing.assert_array_equal(bits16(out.contiguous()), ref)
    if pad:  # the columns past n are never written
        assert torch.isnan(big[:, n:].float()).all()


def _fp8_cases(count: int = 16, seed: int = 4862):
    out = []
    for m, n, k, a_tiled, b_tiled, bias, pad in _cases(64, seed):
        if len(out) < count and m * n * k <= 1.5e8:
            out.append((m, n, k, a_tiled, b_tiled, bias, pad))
    return out


@pytest.mark.parametrize("m,n,k,a_tiled,b_tiled,bias,pad", _fp8_cases())
def test_e4m3_sweep_matches_instruction_model(ops, oracle, device, m, n, k, a_tiled, b_tiled, bias, pad):
    """e4m3 codes bit-exact; outputs against the oracle's model of the FP8
    matrix instruction, to the bound of test_gpu_gemm's fp8 tests."""
    from test_gpu_gemm import _assert_fp8_close

    print(f"e4m3 sweep {m}x{n}x{k} a_tiled={a_tiled} b_tiled={b_tiled} bias={bias} ldo=n+{pad}", flush=True)
    x = activations(m, k, seed=m + k, outlier_channels=max(1, k // 100), outlier_scale=15.0)
    w = weights(n, k, seed=n + k)
    xg, wg = x.to(device), w.to(device)
    qw, sw = (ops.quant_rows_tiled if b_tiled else ops.quant_rows)(wg, ops.FMT_E4M3FN)
    qa, sa = (ops.quant_rows_tiled if a_tiled else ops.quant_rows)(xg, ops.FMT_E4M3FN)
    bvec = (torch.randn(n, generator=torch.Generator().manual_seed(n)) * 0.01).to(torch.bfloat16)
    big = torch.full((m, n + pad), float("nan"), device=device, dtype=torch.bfloat16)
    out = big[:, :n]
    ops.scaled_mm(qa, qw, sa.reshape(-1), sw.reshape(-1), bias=bvec.to(device) if bias else None, out=out,
                  a_tiled=a_tiled, b_tiled=b_tiled, m=m, n=n)
    torch.cuda.synchronize()
    rqa, rsa = oracle.quant_rows(bits16(x), "e4m3")
    rqw, rsw = oracle.quant_rows(bits16(w), "e4m3")
    _assert_fp8_close(oracle, bits16(out.contiguous()), rqa, rsa, rqw, rsw, bits16(bvec) if bias else None)
    if pad:
        assert torch.isnan(big[:, n:].float()).all()


def _lora_cases(count: int = 10, seed: int = 977):
    rng = random.Random(seed)
    out = []
    while len(out) < count:
        m, n, k = rng.randint(129, 700), 8 * rng.randint(1, 90), 128 * rng.randint(1, 12)
        if m * n * k <= 1.5e8:
            out.append((m, n, k, 8 * rng.randint(1, 16), rng.random() < 0.5, rng.random() < 0.5))
    return out


@pytest.mark.parametrize("m,n,k,rank,a_tiled,bias", _lora_cases())
def test_lora_epilogue_layouts_agree(ops, oracle, device, m, n, k, rank, a_tiled, bias):
    """The LoRA epilogue on tiled operands gives the bits of the same call on
    row-major operands, and stays within the reference's rounding points
    (H3/inference/lora_checkpoint.py:196-205) to 2^-7 relative."""
    a_tiled = a_tiled and k >= 256
    print(f"lora sweep {m}x{n}x{k} rank={rank} a_tiled={a_tiled} bias={bias}", flush=True)
    x = activations(m, k, seed=m, outlier_channels=max(1, k // 100), outlier_scale=15.0)
    w = weights(n, k, seed=n)
    gen = torch.Generator().manual_seed(rank)
    la = (torch.randn(rank, k, generator=gen) * 0.01).to(torch.bfloat16)
    lb = (torch.randn(n, rank, generator=gen) * 0.01).to(torch.bfloat16)
    bvec = (torch.randn(n, generator=gen) * 0.01).to(torch.bfloat16)
    xg, wg = x.to(device), w.to(device)
    t = ops.lora_down(xg, la.to(device))
    kw = dict(bias=bvec.to(device) if bias else None, lora_t=t, lora_b=lb.to(device), lora_scale=1.0)
    qa, sa = ops.quant_rows(xg, ops.FMT_E4M3FN)
    qw, sw = ops.quant_rows(wg, ops.FMT_E4M3FN)
    rows = ops.scaled_mm(qa, qw, sa.reshape(-1), sw.reshape(-1), **kw)
    qwt, swt = ops.quant_rows_tiled(wg, ops.FMT_E4M3FN)
    qat, sat = ops.quant_rows_tiled(xg, ops.FMT_E4M3FN) if a_tiled else (qa, sa)
    tiled = ops.scaled_mm(qat, qwt, sat.reshape(-1), swt.reshape(-1), a_tiled=a_tiled, b_tiled=True, m=m, n=n, **kw)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits16(tiled), bits16(rows))
    base = oracle.epilogue(oracle.gemm_e4m3_mfma(bits8(qa), bits8(qw))[0], sa.cpu().numpy(), sw.cpu().numpy(),
                           bits16(bvec) if bias else None)
    ref = oracle.bf16_to_f32(oracle.lora_reference(bits16(x), bits16(la), bits16(lb), 1.0, base)).astype(np.float64)
    got = oracle.bf16_to_f32(bits16(rows)).astype(np.float64)
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 2.0 ** -7
