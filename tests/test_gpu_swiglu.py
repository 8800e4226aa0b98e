"""GPU parity of the fused SwiGLU (+ per-token quantization) producer of the
fc2 input (h3q_swiglu_quant) against the CPU oracle: bf16 rows bit-exact
(orc_swiglu restates the kernel's exp), codes and scales bit-exact as the
pinned quantizer applied to those rows.  Also: torch's eager F.silu(gate) * up
on the same GPU within the stated tolerance (1 bf16 ulp, >= 99.9% identical),
the module mirrors feeding the int8 and per-token FP8 linears, and the host
checks.

Widths cover every register-width variant (half 8 .. 16384, including the
H3 FFN width 14336), ragged row counts, strided rows and special values."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _util import bits8, bits16

pytestmark = pytest.mark.gpu

FMTS = [("int8", "rcp"), ("e4m3", "div"), ("int8", "div")]


def _inputs(rows, half, seed, spread=4.0):
    gen = torch.Generator().manual_seed(seed)
    g = torch.randn(rows, half, generator=gen) * spread
    u = torch.randn(rows, half, generator=gen)
    return torch.cat([g, u], dim=1).to(torch.bfloat16)


def _fmt(ops, fmt, rounding):
    return (ops.FMT_E4M3FN if fmt == "e4m3" else ops.FMT_INT8), (ops.ROUND_DIV if rounding == "div"
                                                                  else ops.ROUND_RCP_MUL)


def _check(ops, oracle, device, x, fmt, rounding, want_out=True, want_codes=True):
    rows, width = x.shape
    print(f"swiglu rows={rows} half={width // 2} {fmt}/{rounding} out={want_out} codes={want_codes}", flush=True)
    f, r = _fmt(ops, fmt, rounding)
    out, codes, scales = ops.swiglu_quant(x.to(device), fmt=f if want_codes else None, rounding=r, out=want_out)
    torch.cuda.synchronize()
    ry = oracle.swiglu(bits16(x))
    if want_out:
        np.testing.assert_array_equal(bits16(out), ry)
    else:
        assert out is None
    if want_codes:
        rq, rs = oracle.quant_rows(ry, fmt, rounding)
        np.testing.assert_array_equal(scales.cpu().numpy().ravel().view(np.uint32), rs.view(np.uint32))
        np.testing.assert_array_equal(bits8(codes), rq.view(np.uint8))


@pytest.mark.parametrize("fmt,rounding", FMTS)
@pytest.mark.parametrize("rows,half", [(64, 1024), (37, 5376), (9, 7168), (5, 14336), (3, 16384), (130, 2048),
                                       (2, 8), (17, 1000), (9, 13824),
                                       # 1024 rows and more: the table form (s looked up per gate pattern)
                                       (1024, 1024), (1061, 13824), (1030, 14336)])
def test_swiglu_matches_oracle(ops, oracle, device, fmt, rounding, rows, half):
    _check(ops, oracle, device, _inputs(rows, half, seed=rows + half), fmt, rounding)


def test_codes_only_output_only_and_strided_rows(ops, oracle, device):
    _check(ops, oracle, device, _inputs(40, 3072, 5), "int8", "rcp", want_out=False)
    _check(ops, oracle, device, _inputs(40, 3072, 6), "int8", "rcp", want_codes=False)
    wide = _inputs(23, 2048 + 32, 7)  # rows of a wider buffer: [gate | up] are its first 2 * 1024 columns
    x = wide[:, :2048]
    out, codes, scales = ops.swiglu_quant(wide.to(device)[:, :2048], fmt=ops.FMT_E4M3FN, out=True)
    torch.cuda.synchronize()
    ry = oracle.swiglu(bits16(x))
    np.testing.assert_array_equal(bits16(out), ry)
    rq, _ = oracle.quant_rows(ry, "e4m3", "div")
    np.testing.assert_array_equal(bits8(codes), rq)


def test_table_form_strided_rows(ops, oracle, device):
    """1030 rows (the table form) read from a wider buffer and written into
    row slices of wider output and code buffers: bit-exact."""
    half = 1024
    wide = _inputs(1030, 2 * half + 64, 8)
    x = wide[:, :2 * half]
    out_wide = torch.zeros(1030, half + 32, device=device, dtype=torch.bfloat16)
    codes_wide = torch.zeros(1030, half + 64, device=device, dtype=torch.float8_e4m3fn)
    scales = torch.empty(1030, 1, device=device, dtype=torch.float32)
    print("swiglu table form, strided rows", flush=True)
    ops.swiglu_quant(wide.to(device)[:, :2 * half], fmt=ops.FMT_E4M3FN, out=out_wide[:, :half],
                     codes=codes_wide[:, :half], scales=scales)
    torch.cuda.synchronize()
    ry = oracle.swiglu(bits16(x))
    np.testing.assert_array_equal(bits16(out_wide[:, :half]), ry)
    assert not bits16(out_wide[:, half:]).any()
    rq, rs = oracle.quant_rows(ry, "e4m3", "div")
    np.testing.assert_array_equal(bits8(codes_wide[:, :half]), rq)
    assert not bits8(codes_wide[:, half:]).any()
    np.testing.assert_array_equal(scales.cpu().numpy().ravel(), rs)


def test_special_values(ops, oracle, device):
    """Zero, huge and infinite gates, gates whose exp overflows, -0 and
    products in the binary32 subnormal range: bit-exact against the oracle."""
    half = 64
    g = torch.zeros(4, half)
    u = torch.ones(4, half)
    g[0, :8] = torch.tensor([0.0, -0.0, 20.0, 1000.0, -100.0, -3e38, float("inf"), -88.5])
    g[1, :8] = torch.tensor([-80.0, -88.0, -89.0, 17.0, -17.0, 1e-30, -1e-30, 3e38])
    u[1, :8] = torch.tensor([1e-5, 1e-5, 1.0, 1e-38, 1e-38, 1.0, 1.0, 1.0])
    g[2] = torch.linspace(-20, 20, half)
    g[3] = torch.linspace(-0.01, 0.01, half)
    x = torch.cat([g, u], 1).to(torch.bfloat16)
    out, _, _ = ops.swiglu_quant(x.to(device), out=True)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits16(out), oracle.swiglu(bits16(x)))


@pytest.mark.parametrize("rows", [64, 1024])
def test_every_bf16_gate(ops, oracle, device, rows):
    """silu depends on the gate alone, so the 65536 bf16 gate values (NaNs,
    infinities, subnormals and both zeros included) with up = 1 cover it
    completely: y = bf16(silu(gate)) bit-exact against the oracle, whose exp
    is the IEEE-only restatement while the kernel uses the hardware exp2.
    NaN gates must give NaN (the payload is not compared).  64 rows run the
    direct form; 1024 rows the table form, whose device table this covers
    entry by entry."""
    gate = np.arange(65536, dtype=np.uint32).astype(np.uint16).reshape(rows, 65536 // rows)
    up = np.full(gate.shape, 0x3F80, dtype=np.uint16)  # bf16 1.0
    xb = np.concatenate([gate, up], axis=1)
    x = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16)
    print(f"swiglu every bf16 gate ({rows} rows, up = 1)", flush=True)
    out, _, _ = ops.swiglu_quant(x.to(device), out=True)
    torch.cuda.synchronize()
    got, want = bits16(out), oracle.swiglu(xb)
    nan_got, nan_want = (got & 0x7FFF) > 0x7F80, (want & 0x7FFF) > 0x7F80
    np.testing.assert_array_equal(nan_got, nan_want)
    np.testing.assert_array_equal(np.where(nan_want, 0, got), np.where(nan_want, 0, want))


def test_torch_eager_on_the_gpu_within_tolerance(ops, device):
    """The reference's eager expression F.silu(gate) * up evaluated by torch on
    the same GPU (its own exp): every output within 1 bf16 ulp, >= 99.9% identical."""
    x = _inputs(256, 5376, 8).to(device)
    out, _, _ = ops.swiglu_quant(x, out=True)
    ref = torch.nn.functional.silu(x[:, :5376]) * x[:, 5376:]
    torch.cuda.synchronize()
    a = bits16(out).astype(np.int32)
    b = bits16(ref).astype(np.int32)
    a = np.where(a & 0x8000, 0x8000 - a, a)
    b = np.where(b & 0x8000, 0x8000 - b, b)
    d = np.abs(a - b)
    assert d.max() <= 1
    assert (d == 0).mean() > 0.999


def test_module_mirrors_and_w8a8_consumers(ops, oracle, device):
    """fused_swiglu keeps the reference's signature; fused_swiglu_w8a8 hands
    codes to cutlass_w8a8_linear (int8) and to the per-token FP8 linear, whose
    outputs equal the unfused path bit for bit."""
    from taomate_h3_amd.distributed.linear import _fp8_w8a8_linear
    from taomate_h3_amd.inference import fused_kernels as fk
    from taomate_h3_amd.inference import w8a8

    tokens, half, n = 96, 1024, 512
    x = _inputs(tokens, half, 9).reshape(2, tokens // 2, 2 * half).to(device)
    y = fk.fused_swiglu(x)
    torch.cuda.synchronize()
    assert tuple(y.shape) == (2, tokens // 2, half)
    np.testing.assert_array_equal(bits16(y.reshape(-1, half)), oracle.swiglu(bits16(x.reshape(-1, 2 * half))))

    w = (torch.randn(n, half, generator=torch.Generator().manual_seed(10)) * 0.02).to(torch.bfloat16).to(device)
    qw, sw = ops.quant_rows_tiled(w, ops.FMT_INT8, ops.ROUND_DIV)
    ops.mark_tiled(qw)
    qa = fk.fused_swiglu_w8a8(x)
    fused = w8a8.cutlass_w8a8_linear(qa, qw, sw, bias=None, workspace=None, weight_t=None, weight_scale_t=None)
    unfused = w8a8.cutlass_w8a8_linear(y, qw, sw, bias=None, workspace=None, weight_t=None, weight_scale_t=None)
    torch.cuda.synchronize()
    assert tuple(fused.shape) == (2, tokens // 2, n)
    np.testing.assert_array_equal(bits16(fused), bits16(unfused))

    qw8, sw8 = ops.quant_rows_tiled(w, ops.FMT_E4M3FN)
    ops.mark_tiled(qw8)
    qa8 = fk.fused_swiglu_w8a8(x, fmt=ops.FMT_E4M3FN, keep_dense=True)
    fused8 = _fp8_w8a8_linear(qa8, qw8, sw8, None)
    unfused8 = _fp8_w8a8_linear(y, qw8, sw8, None)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits16(fk.as_dense(qa8)), bits16(y))
    np.testing.assert_array_equal(bits16(fused8), bits16(unfused8))


def test_host_checks(ops, device):
    with pytest.raises(RuntimeError, match="multiple of 8"):
        ops.swiglu_quant(torch.zeros(2, 2 * 12, dtype=torch.bfloat16, device=device), out=True)
    with pytest.raises(RuntimeError, match="above 16384"):
        ops.swiglu_quant(torch.zeros(1, 2 * 16392, dtype=torch.bfloat16, device=device), out=True)
    with pytest.raises(ValueError, match="neither"):
        ops.swiglu_quant(torch.zeros(2, 32, dtype=torch.bfloat16, device=device))
    with pytest.raises(RuntimeError, match="division form"):
        ops.swiglu_quant(torch.zeros(2, 32, dtype=torch.bfloat16, device=device), fmt=ops.FMT_E4M3FN,
                         rounding=ops.ROUND_RCP_MUL)
