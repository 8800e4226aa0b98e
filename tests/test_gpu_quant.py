"""GPU parity of the quantizers against the CPU oracle (bit-exact codes and scales).

Covers the per-row kernel (vector path and general path), the per-tensor
two-pass kernel, every bf16 value through the e4m3fn conversion, zero rows,
signed zeros, ragged K, row tails and the BASELINE.json full-size activations."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _util import activations, bits8, bits16, from_bits16, weights

pytestmark = pytest.mark.gpu

FMTS = [("e4m3", "div"), ("int8", "div"), ("int8", "rcp")]


def _run_rows(ops, x, fmt, rounding):
    f = ops.FMT_E4M3FN if fmt == "e4m3" else ops.FMT_INT8
    r = ops.ROUND_DIV if rounding == "div" else ops.ROUND_RCP_MUL
    q, s = ops.quant_rows(x, f, r)
    torch.cuda.synchronize()
    return bits8(q), s.cpu().numpy().ravel()


def _check_rows(ops, oracle, x_cpu, device, fmt, rounding):
    xb = bits16(x_cpu)
    q, s = _run_rows(ops, x_cpu.to(device), fmt, rounding)
    rq, rs = oracle.quant_rows(xb, fmt, rounding)
    np.testing.assert_array_equal(s.view(np.uint32), rs.view(np.uint32))
    np.testing.assert_array_equal(q, rq.view(np.uint8))


@pytest.mark.parametrize("fmt,rounding", FMTS)
@pytest.mark.parametrize("m,k", [(256, 1024), (61, 5120), (5, 13824), (3, 1000), (2, 20000), (1, 8), (9, 7)])
def test_rows_match_oracle(ops, oracle, device, fmt, rounding, m, k):
    print(f"rows {fmt}/{rounding} m={m} k={k}", flush=True)
    x = activations(m, k, seed=m * 131 + k, outlier_channels=max(1, k // 100), outlier_scale=15.0)
    _check_rows(ops, oracle, x, device, fmt, rounding)


@pytest.mark.parametrize("fmt,rounding", FMTS)
def test_rows_strided_input(ops, oracle, device, fmt, rounding):
    """A column slice of a wider matrix (leading dimension > K)."""
    wide = activations(33, 2048 + 64, seed=5)
    x = wide[:, 32:32 + 2048]
    f = ops.FMT_E4M3FN if fmt == "e4m3" else ops.FMT_INT8
    r = ops.ROUND_DIV if rounding == "div" else ops.ROUND_RCP_MUL
    q, s = ops.quant_rows(wide.to(device)[:, 32:32 + 2048], f, r)
    torch.cuda.synchronize()
    rq, rs = oracle.quant_rows(bits16(x), fmt, rounding)
    np.testing.assert_array_equal(bits8(q), rq.view(np.uint8))
    np.testing.assert_array_equal(s.cpu().numpy().ravel(), rs)


def test_e4m3_conversion_every_bf16_value(ops, oracle, device):
    """Rows whose amax is 448 have scale exactly 1, so every other element's
    code is e4m3fn(x): this puts every bf16 value in [-448, 448] (both signs,
    subnormals and signed zeros) through the device conversion."""
    bits = np.arange(0, 0x8000, dtype=np.uint16)
    vals = oracle.bf16_to_f32(bits)
    keep = bits[np.isfinite(vals) & (vals <= 448.0)]
    allv = np.concatenate([keep, keep | 0x8000]).astype(np.uint16)
    k = 1023
    pad = (-allv.size) % k
    allv = np.concatenate([allv, np.zeros(pad, dtype=np.uint16)])
    body = allv.reshape(-1, k)
    col448 = np.full((body.shape[0], 1), oracle.f32_to_bf16(np.array([448.0], dtype=np.float32))[0], dtype=np.uint16)
    xb = np.concatenate([body, col448], axis=1)
    x = from_bits16(xb)
    q, s = _run_rows(ops, x.to(device), "e4m3", "div")
    assert np.all(s == 1.0)
    rq, _ = oracle.quant_rows(xb, "e4m3")
    np.testing.assert_array_equal(q, rq)
    direct = oracle.f32_to_e4m3(oracle.bf16_to_f32(xb[:64]))
    np.testing.assert_array_equal(rq[:64], direct)


@pytest.mark.parametrize("fmt,rounding", FMTS)
def test_zero_and_signed_zero_rows(ops, oracle, device, fmt, rounding):
    x = torch.zeros(6, 640, dtype=torch.bfloat16)
    x[1] = -0.0
    x[2, 5] = -0.0
    x[3, 7] = 3.0
    x[4, ::2] = -0.0
    x[5, 100] = 1e-39  # bf16 subnormal
    _check_rows(ops, oracle, x, device, fmt, rounding)


@pytest.mark.parametrize("fmt,rounding", FMTS)
def test_rows_extreme_magnitudes(ops, oracle, device, fmt, rounding):
    gen = torch.Generator().manual_seed(7)
    x = torch.randn(16, 512, generator=gen)
    x *= torch.logspace(-30, 30, 16).unsqueeze(1)
    x[0, :] = 1e-38
    x[1, 3] = 3.0e38
    _check_rows(ops, oracle, x.to(torch.bfloat16), device, fmt, rounding)


def _special_rows(k: int) -> torch.Tensor:
    """Rows holding infinities and NaNs among finite values (and one plain
    row): an infinite amax makes the scale infinite, a NaN amax makes it NaN."""
    gen = torch.Generator().manual_seed(11)
    x = torch.randn(6, k, generator=gen)
    x[0, 17] = float("inf")
    x[1, 3] = float("-inf")
    x[1, 5] = float("inf")
    x[2, 40] = float("nan")
    x[3, 0] = float("nan")
    x[3, k - 1] = float("inf")
    x[5, :] = float("inf")
    return x.to(torch.bfloat16)


def _check_special(q, s, rq, rs, fmt):
    """Codes equal the oracle's, NaN codes compared as NaN (their sign bit is
    not fixed by the reference: the sign of x / s for a NaN s is unspecified);
    scales equal bit for bit, NaN scales as NaN."""
    nan_s = np.isnan(rs)
    np.testing.assert_array_equal(np.isnan(s), nan_s)
    np.testing.assert_array_equal(s[~nan_s], rs[~nan_s])
    if fmt == "e4m3":
        want = rq.view(np.uint8)
        nan_q = (want & 0x7F) == 0x7F
        np.testing.assert_array_equal((q & 0x7F) == 0x7F, nan_q)
        np.testing.assert_array_equal(np.where(nan_q, 0, q), np.where(nan_q, 0, want))
    else:
        np.testing.assert_array_equal(q, rq.view(np.uint8))


@pytest.mark.parametrize("fmt,rounding", [("e4m3", "div"), ("int8", "div")])
@pytest.mark.parametrize("k", [640, 5120, 1000])
def test_rows_with_infinities_and_nans(ops, oracle, device, fmt, rounding, k):
    """x / s with s = inf is +-0 for finite x and NaN for x = +-inf (IEEE
    division, the reference's torch expression); a NaN in the row gives a NaN
    scale and NaN quotients.  Row-major (vector and general kernels) and
    tiled codes."""
    from _util import from_tiled

    print(f"rows with inf / nan {fmt} k={k}", flush=True)
    x = _special_rows(k)
    xb = bits16(x)
    rq, rs = oracle.quant_rows(xb, fmt, rounding)
    q, s = _run_rows(ops, x.to(device), fmt, rounding)
    _check_special(q, s, rq, rs, fmt)
    if k % 128 == 0:
        f = ops.FMT_E4M3FN if fmt == "e4m3" else ops.FMT_INT8
        qt, st = ops.quant_rows_tiled(x.to(device), f, ops.ROUND_DIV)
        torch.cuda.synchronize()
        _check_special(from_tiled(bits8(qt), qt.shape[0], k)[:x.shape[0]], st.cpu().numpy().ravel(), rq, rs, fmt)


@pytest.mark.parametrize("fmt", ["e4m3", "int8"])
def test_rows_with_infinities_and_nans_match_the_reference_on_the_gpu(ops, device, fmt):
    """The same rows through the reference's own torch expressions evaluated
    on this GPU (H3/inference/w8a8.py:57-63 and its e4m3 counterpart): equal
    codes and scales, NaN codes compared as NaN; for int8, positions whose
    quotient is NaN are left out (torch's float -> int8 cast of a NaN is not
    defined)."""
    from oracle import torch_path as TP

    xd = _special_rows(1024).to(device)
    if fmt == "e4m3":
        tq, ts = TP.quantize_rows_e4m3(xd)
        q, s = ops.quant_rows(xd, ops.FMT_E4M3FN, ops.ROUND_DIV)
    else:
        tq, ts = TP.quantize_weight_int8(xd)
        q, s = ops.quant_rows(xd, ops.FMT_INT8, ops.ROUND_DIV)
    torch.cuda.synchronize()
    got_s, want_s = s.cpu().numpy().ravel(), ts.cpu().numpy().ravel()
    np.testing.assert_array_equal(np.isnan(got_s), np.isnan(want_s))
    np.testing.assert_array_equal(got_s[~np.isnan(want_s)], want_s[~np.isnan(want_s)])
    got, want = bits8(q), bits8(tq)
    if fmt == "e4m3":
        skip = (want & 0x7F) == 0x7F
        np.testing.assert_array_equal((got & 0x7F) == 0x7F, skip)
    else:
        skip = torch.isnan(xd.float() / ts).cpu().numpy()
    np.testing.assert_array_equal(np.where(skip, 0, got), np.where(skip, 0, want))


# Shapes include the c2 activations (8192 x 5120) and row counts past the
# 1024-workgroup grid of the two passes (several rows per wave).
@pytest.mark.parametrize("static", [False, True])
@pytest.mark.parametrize("m,k", [(256, 1024), (1000, 5120), (3, 37), (4097, 8), (8192, 5120), (9000, 256),
                                 (8200, 5120), (16400, 64)])
def test_tensor_e4m3_matches_oracle(ops, oracle, device, static, m, k):
    x = activations(m, k, seed=m + k, outlier_channels=max(1, k // 100))
    xb = bits16(x)
    st = 0.0371 if static else None
    sg = torch.tensor(st, dtype=torch.float32, device=device) if static else None
    q, s = ops.quant_tensor_e4m3(x.to(device), sg)
    torch.cuda.synchronize()
    rq, rs = oracle.quant_tensor_e4m3(xb, st)
    assert np.float32(s.item()) == rs
    np.testing.assert_array_equal(bits8(q), rq)


@pytest.mark.parametrize("static", [False, True])
@pytest.mark.parametrize("m,k", [(1000, 5120), (3, 37), (8192, 5120), (8200, 5120)])
def test_tensor_e4m3_bf16_divisor_matches_oracle(ops, oracle, device, static, m, k):
    """The eager-on-GPU form (h3q_quant_tensor_e4m3_bf16_divisor): divisor
    bf16(s), returned scale s."""
    x = activations(m, k, seed=m + k + 1, outlier_channels=max(1, k // 100))
    st = 0.0371 if static else None
    sg = torch.tensor(st, dtype=torch.float32, device=device) if static else None
    q, s = ops.quant_tensor_e4m3(x.to(device), sg, bf16_divisor=True)
    torch.cuda.synchronize()
    rq, rs = oracle.quant_tensor_e4m3(bits16(x), st, bf16_divisor=True)
    assert np.float32(s.item()) == rs
    np.testing.assert_array_equal(bits8(q), rq)


@pytest.mark.parametrize("case", ["inf", "nan", "static"])
@pytest.mark.parametrize("bf16_divisor", [False, True])
def test_tensor_e4m3_infinities_and_nans(ops, oracle, device, case, bf16_divisor):
    """An infinity in the tensor makes the dynamic scale infinite (finite
    elements -> +-0, infinite ones -> NaN); a NaN makes it NaN (every code
    NaN); under a static scale an infinity saturates to +-448 and a NaN stays
    NaN (torch.clamp keeps it; v_med3 alone would give -448).  NaN codes are
    compared as NaN (their sign is not fixed by the reference)."""
    x = activations(1000, 5120, seed=21)
    if case in ("inf", "static"):
        x[3, 17] = float("inf")
        x[999, 5119] = float("-inf")
    if case in ("nan", "static"):
        x[500, 2] = float("nan")
    xb = bits16(x)
    st = 0.0371 if case == "static" else None
    sg = torch.tensor(st, dtype=torch.float32, device=device) if st else None
    q, s = ops.quant_tensor_e4m3(x.to(device), sg, bf16_divisor=bf16_divisor)
    torch.cuda.synchronize()
    rq, rs = oracle.quant_tensor_e4m3(xb, st, bf16_divisor=bf16_divisor)
    s = np.float32(s.item())
    assert (np.isnan(s) and np.isnan(rs)) or s == rs
    got, want = bits8(q), rq.view(np.uint8)
    nan_q = (want & 0x7F) == 0x7F
    np.testing.assert_array_equal((got & 0x7F) == 0x7F, nan_q)
    np.testing.assert_array_equal(np.where(nan_q, 0, got), np.where(nan_q, 0, want))
    if case == "static":
        assert got[3, 17] == 0x7E and got[999, 5119] == 0xFE


def test_tensor_e4m3_3d_input(ops, oracle, device):
    x = activations(2 * 48, 256, seed=3).reshape(2, 48, 256)
    q, s = ops.quant_tensor_e4m3(x.to(device))
    torch.cuda.synchronize()
    rq, rs = oracle.quant_tensor_e4m3(bits16(x.reshape(-1, 256)))
    assert tuple(q.shape) == (2, 48, 256)
    np.testing.assert_array_equal(bits8(q).reshape(-1, 256), rq)
    assert np.float32(s.item()) == rs


@pytest.mark.parametrize("name,m,k,fmt,rounding,student", [
    ("c2_qkv_480p", 8192, 5120, "e4m3", "div", False),
    ("c3_down_in", 2048, 13824, "e4m3", "div", False),
    ("c5_int8_1080p", 40960, 5120, "int8", "rcp", True),
])
def test_full_size_activations(ops, oracle, device, name, m, k, fmt, rounding, student):
    """BASELINE.json activation shapes (c3 down: 2048 of its 24576 rows), bit-exact."""
    print(f"full-size act quant {name}", flush=True)
    x = activations(m, k, seed=0, outlier_channels=max(1, k // 100), outlier_scale=15.0, student_t=student)
    _check_rows(ops, oracle, x, device, fmt, rounding)


@pytest.mark.parametrize("fmt,rounding", [("e4m3", "div"), ("int8", "div"), ("int8", "rcp")])
@pytest.mark.parametrize("n,k,chunk", [(64, 512, 64), (96, 1024, 40), (48, 5120, 7), (16, 128, 16),
                                       (80, 5376, 48), (32, 13824, 32), (64, 7168, 50), (48, 640, 16),
                                       (64, 16384, 32)])
def test_tiled_quantizer_matches_permuted_oracle(ops, oracle, device, fmt, rounding, n, k, chunk):
    """h3q_quant_rows_tiled in row chunks (any chunk size, like the streamed
    loader) == the oracle's row-major codes permuted into the tiled layout."""
    from _util import to_tiled

    w = weights(n, k, seed=n + k)
    f = ops.FMT_E4M3FN if fmt == "e4m3" else ops.FMT_INT8
    r = ops.ROUND_DIV if rounding == "div" else ops.ROUND_RCP_MUL
    codes = torch.zeros((n, k), device=device, dtype=ops.code_dtype(f))
    scales = torch.empty((n, 1), device=device, dtype=torch.float32)
    wg = w.to(device)
    for r0 in range(0, n, chunk):
        r1 = min(n, r0 + chunk)
        ops.quant_rows_tiled(wg[r0:r1], f, r, codes=codes, row0=r0, scales=scales[r0:r1])
    torch.cuda.synchronize()
    rq, rs = oracle.quant_rows(bits16(w), fmt, rounding)
    np.testing.assert_array_equal(bits8(codes), to_tiled(rq.view(np.uint8)))
    np.testing.assert_array_equal(scales.cpu().numpy().ravel(), rs)


@pytest.mark.parametrize("m,k,fmt,rounding", [(8192, 5120, "e4m3", "div"), (4100, 13824, "e4m3", "div"),
                                               (2064, 5120, "int8", "rcp")])
def test_tiled_activations_full_size(ops, oracle, device, m, k, fmt, rounding):
    """Activation codes written straight into the tiled layout by whole
    16-row blocks (plus a ragged tail), at the c2 / c3-down / c5 widths."""
    from _util import from_tiled

    print(f"tiled act quant {m}x{k} {fmt}", flush=True)
    x = activations(m, k, seed=m, outlier_channels=max(1, k // 100), outlier_scale=15.0)
    f = ops.FMT_E4M3FN if fmt == "e4m3" else ops.FMT_INT8
    r = ops.ROUND_DIV if rounding == "div" else ops.ROUND_RCP_MUL
    q, s = ops.quant_rows_tiled(x.to(device), f, r)
    torch.cuda.synchronize()
    rq, rs = oracle.quant_rows(bits16(x), fmt, rounding)
    # rows past m are padding of the last block: compare the real rows
    np.testing.assert_array_equal(from_tiled(bits8(q), q.shape[0], k)[:m], rq.view(np.uint8))
    np.testing.assert_array_equal(s.cpu().numpy().ravel(), rs)


def test_int8_rcp_known_answers(ops, device):
    """The vLLM-form kernel (h3q_quant_rows INT8 + RCP_MUL) against closed-form
    known answers evaluated in exact rational arithmetic (tests/_exact32.py):
    the half-integer ties where the reciprocal-multiply and division forms
    disagree, +-amax -> +-127, and a zero row."""
    import _exact32 as E

    cases = E.separating_cases()
    k = 64
    rows = np.zeros((len(cases) + 1, k), dtype=np.float32)
    for r, (x, amax, _, _) in enumerate(cases):
        rows[r, 0], rows[r, 1], rows[r, 2], rows[r, 3] = amax, x, -x, -amax
    x = torch.from_numpy(rows).to(torch.bfloat16)
    q, s = _run_rows(ops, x.to(device), "int8", "rcp")
    q = q.view(np.int8)
    for r, (xv, amax, q_rcp, q_div) in enumerate(cases):
        assert (q[r, 1], q[r, 2]) == (q_rcp, -q_rcp), (xv, amax, q[r, 1], q_rcp)
        assert q[r, 1] != q_div
        assert (q[r, 0], q[r, 3]) == (127, -127)
        assert s[r] == np.float32(float(E.int8_scale(amax)))
    assert s[-1] == 0.0 and not q[-1].any()
