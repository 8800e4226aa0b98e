"""GPU parity of the fused RMSNorm + AdaLN modulate (+ residual gate) +
per-token quantization kernel against the CPU oracle: bf16 outputs, hidden
rows, codes and scales bit-exact.  The codes are also checked as the
composition oracle.quant_rows(oracle.rms_norm_modulate(...)), i.e. against
the already pinned quantizer applied to the pinned modulated rows.

Covers every register-width variant of the kernel (cols 8 .. 8192), ragged
row counts, several table rows selected per row, strided inputs, outputs
without codes and codes without outputs, and the module-level mirrors
(fused_rms_norm_modulate, fused_residual_gate_rms_norm_modulate and their
W8A8 variants feeding cutlass_w8a8_linear / the FP8 linear)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _util import activations, bits8, bits16, from_bits16

pytestmark = pytest.mark.gpu

FMTS = [("int8", "rcp"), ("e4m3", "div"), ("int8", "div")]


def _tables(t: int, cols: int, seed: int, spread: float = 0.2):
    gen = torch.Generator().manual_seed(seed)
    scale = (torch.randn(t, cols, generator=gen) * spread).to(torch.bfloat16)
    shift = (torch.randn(t, cols, generator=gen) * spread).to(torch.bfloat16)
    gate = (torch.randn(t, cols, generator=gen) * 0.5 + 1.0).to(torch.bfloat16)
    weight = (1.0 + 0.1 * torch.randn(cols, generator=gen)).to(torch.bfloat16)
    return weight, scale, shift, gate


def _fmt(ops, fmt, rounding):
    return (ops.FMT_E4M3FN if fmt == "e4m3" else ops.FMT_INT8), (ops.ROUND_DIV if rounding == "div"
                                                                  else ops.ROUND_RCP_MUL)


def _check(ops, oracle, device, rows, cols, fmt, rounding, resid, t=3, seed=0, eps=1e-6, want_out=True,
           want_codes=True):
    print(f"norm_quant rows={rows} cols={cols} {fmt}/{rounding} resid={resid} out={want_out} codes={want_codes}",
          flush=True)
    x = activations(rows, cols, seed=seed, outlier_channels=max(1, cols // 128), outlier_scale=12.0)
    branch = activations(rows, cols, seed=seed + 7)
    weight, scale, shift, gate = _tables(t, cols, seed + 1)
    idx = torch.randint(0, t, (rows,), generator=torch.Generator().manual_seed(seed + 2), dtype=torch.int64)
    f, r = _fmt(ops, fmt, rounding)
    hidden = torch.empty(rows, cols, device=device, dtype=torch.bfloat16) if resid else None
    rg = (branch.to(device), gate.to(device), hidden) if resid else None
    out, codes, scales = ops.norm_modulate_quant(
        x.to(device), weight.to(device), scale.to(device), shift.to(device), idx.to(device), eps,
        fmt=f if want_codes else None, rounding=r, out=want_out, residual_gate=rg)
    torch.cuda.synchronize()
    ry, rh = oracle.rms_norm_modulate(bits16(x), bits16(weight), bits16(scale), bits16(shift), idx.numpy(), eps,
                                      residual_gate=(bits16(branch), bits16(gate)) if resid else None)
    if resid:
        np.testing.assert_array_equal(bits16(hidden), rh)
    if want_out:
        np.testing.assert_array_equal(bits16(out), ry)
    else:
        assert out is None
    if want_codes:
        rq, rs = oracle.quant_rows(ry, fmt, rounding)
        np.testing.assert_array_equal(scales.cpu().numpy().ravel().view(np.uint32), rs.view(np.uint32))
        np.testing.assert_array_equal(bits8(codes), rq.view(np.uint8))


@pytest.mark.parametrize("fmt,rounding", FMTS)
@pytest.mark.parametrize("resid", [False, True])
@pytest.mark.parametrize("rows,cols", [(64, 1024), (37, 5120), (19, 5376), (5, 8192), (9, 1000), (3, 8), (130, 2048)])
def test_fused_matches_oracle(ops, oracle, device, fmt, rounding, resid, rows, cols):
    _check(ops, oracle, device, rows, cols, fmt, rounding, resid, seed=rows * 31 + cols)


@pytest.mark.parametrize("resid", [False, True])
def test_codes_only_and_output_only(ops, oracle, device, resid):
    _check(ops, oracle, device, 40, 3072, "int8", "rcp", resid, want_out=False, seed=11)
    _check(ops, oracle, device, 40, 3072, "int8", "rcp", resid, want_codes=False, seed=12)


def test_strided_rows_and_table(ops, oracle, device):
    """value rows with a leading dimension above cols; a table whose rows are
    a column slice of a wider tensor."""
    rows, cols, t = 23, 2048, 4
    wide = activations(rows, cols + 64, seed=3)
    weight, scale_w, shift_w, _ = _tables(t, cols + 64, 4)
    weight = weight[:cols].contiguous()
    idx = torch.tensor([i % t for i in range(rows)], dtype=torch.int64)
    out, codes, scales = ops.norm_modulate_quant(
        wide.to(device)[:, 8:8 + cols], weight.to(device), scale_w.to(device)[:, 16:16 + cols],
        shift_w.to(device)[:, 16:16 + cols], idx.to(device), 1e-5, fmt=ops.FMT_INT8, rounding=ops.ROUND_RCP_MUL,
        out=True)
    torch.cuda.synchronize()
    ry, _ = oracle.rms_norm_modulate(bits16(wide[:, 8:8 + cols]), bits16(weight), bits16(scale_w[:, 16:16 + cols]),
                                     bits16(shift_w[:, 16:16 + cols]), idx.numpy(), 1e-5)
    np.testing.assert_array_equal(bits16(out), ry)
    rq, rs = oracle.quant_rows(ry, "int8", "rcp")
    np.testing.assert_array_equal(bits8(codes), rq.view(np.uint8))


def test_zero_rows_and_special_tables(ops, oracle, device):
    """A zero row normalizes to 0 (rs = 1/sqrt(eps)), so its output is the
    shift row; scale = -1 makes every output the shift exactly."""
    rows, cols = 8, 1024
    x = activations(rows, cols, seed=9)
    x[2] = 0
    weight, scale, shift, _ = _tables(2, cols, 10)
    scale[1] = -1.0
    idx = torch.tensor([0, 0, 0, 1, 1, 0, 1, 0], dtype=torch.int64)
    out, codes, scales = ops.norm_modulate_quant(x.to(device), weight.to(device), scale.to(device), shift.to(device),
                                                 idx.to(device), 1e-6, fmt=ops.FMT_E4M3FN, rounding=ops.ROUND_DIV,
                                                 out=True)
    torch.cuda.synchronize()
    got = bits16(out)
    np.testing.assert_array_equal(got[2], bits16(shift)[0])
    for r in (3, 4, 6):
        np.testing.assert_array_equal(got[r], bits16(shift)[1])
    ry, _ = oracle.rms_norm_modulate(bits16(x), bits16(weight), bits16(scale), bits16(shift), idx.numpy(), 1e-6)
    np.testing.assert_array_equal(got, ry)


def test_module_mirrors_and_w8a8_consumers(ops, oracle, device):
    """fused_* keep the reference's signatures; the *_w8a8 variants hand codes
    to cutlass_w8a8_linear and to the per-token FP8 linear, whose outputs equal
    the unfused path (producer -> bf16 -> act-quant -> GEMM) bit for bit."""
    from taomate_h3_amd.distributed.linear import _fp8_w8a8_linear
    from taomate_h3_amd.inference import fused_kernels as fk
    from taomate_h3_amd.inference import w8a8

    tokens, cols, n, t = 96, 1024, 512, 2
    x = activations(tokens, cols, seed=21).reshape(2, tokens // 2, cols).to(device)
    branch = activations(tokens, cols, seed=22).reshape(2, tokens // 2, cols).to(device)
    weight, scale, shift, gate = (v.to(device) for v in _tables(t, cols, 23))
    idx = torch.tensor([i % t for i in range(tokens)], dtype=torch.int64, device=device).reshape(2, -1)

    y = fk.fused_rms_norm_modulate(x, weight, scale, shift, idx, 1e-6)
    hid, y2 = fk.fused_residual_gate_rms_norm_modulate(x, branch, gate, weight, scale, shift, idx, 1e-6)
    ry, _ = oracle.rms_norm_modulate(bits16(x.reshape(-1, cols)), bits16(weight), bits16(scale), bits16(shift),
                                     idx.reshape(-1).cpu().numpy(), 1e-6)
    np.testing.assert_array_equal(bits16(y.reshape(-1, cols)), ry)
    ry2, rh2 = oracle.rms_norm_modulate(bits16(x.reshape(-1, cols)), bits16(weight), bits16(scale), bits16(shift),
                                        idx.reshape(-1).cpu().numpy(), 1e-6,
                                        residual_gate=(bits16(branch.reshape(-1, cols)), bits16(gate)))
    np.testing.assert_array_equal(bits16(hid.reshape(-1, cols)), rh2)
    np.testing.assert_array_equal(bits16(y2.reshape(-1, cols)), ry2)
    with pytest.raises(ValueError, match="indices do not cover every row"):
        fk.fused_rms_norm_modulate(x, weight, scale, shift, idx[:, :3], 1e-6)

    # int8 W8A8 (tiled weight, as the module stores it)
    w = (torch.randn(n, cols, generator=torch.Generator().manual_seed(24)) * 0.02).to(torch.bfloat16).to(device)
    qw, sw = ops.quant_rows_tiled(w, ops.FMT_INT8, ops.ROUND_DIV)
    ops.mark_tiled(qw)
    qa = fk.fused_rms_norm_modulate_w8a8(x, weight, scale, shift, idx, 1e-6)
    fused = w8a8.cutlass_w8a8_linear(qa, qw, sw, bias=None, workspace=None, weight_t=None, weight_scale_t=None)
    unfused = w8a8.cutlass_w8a8_linear(y, qw, sw, bias=None, workspace=None, weight_t=None, weight_scale_t=None)
    torch.cuda.synchronize()
    assert tuple(fused.shape) == (2, tokens // 2, n)
    np.testing.assert_array_equal(bits16(fused), bits16(unfused))

    # per-token FP8 W8A8 with bias, through the residual-gate producer
    qw8, sw8 = ops.quant_rows_tiled(w, ops.FMT_E4M3FN)
    ops.mark_tiled(qw8)
    bias = (torch.randn(n, generator=torch.Generator().manual_seed(25)) * 0.1).to(torch.bfloat16).to(device)
    hid3, qa8 = fk.fused_residual_gate_rms_norm_modulate_w8a8(x, branch, gate, weight, scale, shift, idx, 1e-6,
                                                              fmt=ops.FMT_E4M3FN, keep_dense=True)
    fused8 = _fp8_w8a8_linear(qa8, qw8, sw8, bias)
    unfused8 = _fp8_w8a8_linear(y2, qw8, sw8, bias)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits16(hid3), bits16(hid))
    np.testing.assert_array_equal(bits16(fk.as_dense(qa8)), bits16(y2))
    np.testing.assert_array_equal(bits16(fused8), bits16(unfused8))
    with pytest.raises(TypeError, match="int8 activation codes"):
        w8a8.cutlass_w8a8_linear(qa8, qw, sw, bias=None, workspace=None, weight_t=None, weight_scale_t=None)


def test_full_size_hidden_5376(ops, oracle, device):
    """The real H3 hidden width (TP-local K = 5376) at 1312 tokens (480p,
    phase 0), int8 codes for the QKV linear."""
    _check(ops, oracle, device, 1312, 5376, "int8", "rcp", True, t=6, seed=77, want_out=False)


def test_more_than_64_rows_per_wave(ops, oracle, device):
    """Past 64 * 4096 rows a wave handles more than 64 rows and re-reads the
    table indices of its next 64 rows; random indices over five table rows
    make a misplaced index visible."""
    _check(ops, oracle, device, 64 * 4096 + 37, 8, "int8", "rcp", resid=True, t=5, seed=11)


@pytest.mark.parametrize("fmt,rounding", [("e4m3", "div"), ("int8", "rcp")])
def test_rows_with_infinities_and_nans(ops, oracle, device, fmt, rounding):
    """Rows holding an infinity, a NaN, values whose squares overflow the sum
    (so rs = 0), and an all-zero row (rs = 1/sqrt(eps)): the normalized,
    modulated rows, codes and scales follow the oracle's IEEE operations;
    NaNs are compared as NaN (their payload and sign are not fixed)."""
    rows, cols, eps = 6, 1024, 1e-6
    x = activations(rows, cols, seed=31)
    x[0, 5] = float("inf")
    x[1, 9] = float("nan")
    x[2, :] = 3.0e38
    x[3, :] = 0.0
    x[5, 7] = float("-inf")
    weight, scale, shift, _ = _tables(2, cols, 32)
    idx = torch.tensor([0, 1, 0, 1, 0, 1], dtype=torch.int64)
    f, r = _fmt(ops, fmt, rounding)
    print(f"norm_quant special rows {fmt}/{rounding}", flush=True)
    out, codes, scales = ops.norm_modulate_quant(x.to(device), weight.to(device), scale.to(device),
                                                 shift.to(device), idx.to(device), eps, fmt=f, rounding=r, out=True)
    torch.cuda.synchronize()
    ry, _ = oracle.rms_norm_modulate(bits16(x), bits16(weight), bits16(scale), bits16(shift), idx.numpy(), eps)
    got = bits16(out)
    nan_y = (ry & 0x7FFF) > 0x7F80
    np.testing.assert_array_equal((got & 0x7FFF) > 0x7F80, nan_y)
    np.testing.assert_array_equal(np.where(nan_y, 0, got), np.where(nan_y, 0, ry))
    rq, rs = oracle.quant_rows(ry, fmt, rounding)
    got_s = scales.cpu().numpy().ravel()
    np.testing.assert_array_equal(np.isnan(got_s), np.isnan(rs))
    np.testing.assert_array_equal(got_s[~np.isnan(rs)], rs[~np.isnan(rs)])
    gq, wq = bits8(codes), rq.view(np.uint8)
    nan_q = ((wq & 0x7F) == 0x7F) if fmt == "e4m3" else np.zeros(wq.shape, dtype=bool)
    if fmt == "e4m3":
        np.testing.assert_array_equal((gq & 0x7F) == 0x7F, nan_q)
    np.testing.assert_array_equal(np.where(nan_q, 0, gq), np.where(nan_q, 0, wq))
